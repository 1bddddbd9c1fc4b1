"""bench.py - libosmos MI355X's headline benchmark on one MI355X.

Headline (value): the Qwen-style 512-expert MoE layer in IQ3_XXS at batch 1 (hidden 2048, expert
ff 512, top-10 of 512) - one step is one routed layer through the C ABI's osmos_lane_layer (round x, device-built
tables, fused gate/up + SwiGLU, round h, down, ascending-expert token sums), bit-exact to the reference CPU lane.
value = algorithmic bytes a step (each distinct routed expert's gate + up + down once, x in, the output out) / time a
step, in GB/s; weights resident in HBM and rotated through more than 2 GiB of layer copies so the 256 MB Infinity Cache
cannot serve them; steps captured in a HIP graph (the decode's launch pattern), timed with events between
synchronizations.

roofline: the dominant kernel (the layer's fused gate/up launch, through osmos_lane_gate_up) timed alone, its
algorithmic bytes a launch over its average duration (events on the launching stream), against MI355X's 8 TB/s; the
down launch's figures beside it.
cpu_baseline: the reference's own CPU path (oracle/_ref: src/cpu/q8.c's cpu_q8_rows and kernels/lane.h) on the host's
cores for the same layer, rows split evenly over the threads as src/cpu/lane.c splits them.

prefill_bs512 (every run): the metric's batch-512 half, config 5's expert GEMMs (int8 TOPS, % of MFMA peak, roofline
fraction). gemv_bs1 (every run): the metric's GEMV half on configs 1 and 2 at one token (Q4_0 2048 -> 8192, Q4_K and
Q3_K 2048 -> 6144: the lane's int8 GEMV and the fp32 matvec, HBM GB/s and % of peak).

--all adds the other BASELINE configs as `extra` lines (Q4_K / Q3_K at 8 and 64 tokens, the Qwen layer at 4 and 32,
the DeepSeek IQ1 experts) - they are reported, not the headline.
"""
import argparse
import ctypes
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0
F16_PEAK_TFLOPS = 2500.0
METRIC = "quant GEMV GB/s (% HBM peak) bs=1; expert GEMM int8 TOPS (% MFMA) bs=512"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


class Events:
    """elapsed ms between two points on the current stream"""

    def __init__(self, torch):
        self.torch = torch

    def time(self, fn, reps):
        t = self.torch
        s = t.cuda.current_stream()
        a, b = t.cuda.Event(enable_timing=True), t.cuda.Event(enable_timing=True)
        t.cuda.synchronize()
        a.record(s)
        for _ in range(reps):
            fn()
        b.record(s)
        t.cuda.synchronize()
        return a.elapsed_time(b)


def iq_weights(torch, gen, n_blocks, block_bytes, d_at=0, sigma=0.02):
    """IQ blocks on the device: uniform random bytes (grid indices, signs, sub-scales), each block's f16 scale
    |N(0, sigma)| at byte d_at (the BASELINE configs' weights)"""
    raw = torch.randint(0, 256, (n_blocks, block_bytes), dtype=torch.uint8, device="cuda", generator=gen)
    d = (torch.randn(n_blocks, device="cuda", generator=gen).abs_() * sigma).half().view(torch.int16).to(torch.int32)
    raw[:, d_at] = (d & 0xFF).to(torch.uint8)
    raw[:, d_at + 1] = ((d >> 8) & 0xFF).to(torch.uint8)
    return raw.reshape(-1)


SCALE_AT = {"Q4_0": [0], "Q8_0": [0], "Q3_K": [108], "Q4_K": [0, 2], "IQ2_XXS": [0], "IQ3_XXS": [0], "IQ1_S": [0]}
BLOCK = {"Q4_0": (32, 18), "Q3_K": (256, 110), "Q4_K": (256, 144), "IQ2_XXS": (256, 66), "IQ3_XXS": (256, 98),
         "IQ1_S": (256, 50), "IQ1_M": (256, 56)}
TYPE_ID = {"Q4_0": 2, "Q3_K": 11, "Q4_K": 12, "IQ2_XXS": 16, "IQ3_XXS": 18, "IQ1_S": 19, "IQ1_M": 29}


def blocks_of(torch, gen, name, rows, cols, copies=1, sigma=0.02):
    """copies x rows x cols of `name` on the device: uniform random bytes (codes, grid indices, signs, sub-scales),
    each block's f16 scale(s) |N(0, sigma)| (IQ1_M's scale nibbles the same f16) - the BASELINE configs' synthetic
    weights. returns uint8 [copies, rows * row bytes]"""
    v, b = BLOCK[name]
    nblk = copies * rows * (cols // v)
    raw = torch.randint(0, 256, (nblk, b), dtype=torch.uint8, device="cuda", generator=gen)
    d = (torch.randn(nblk, device="cuda", generator=gen).abs_() * sigma).half().view(torch.int16).to(torch.int32)
    if name == "IQ1_M":  # the scale's 4 nibbles at the top of the 4 scale words (bytes 49, 51, 53, 55)
        for k in range(4):
            at = 49 + 2 * k
            raw[:, at] = (raw[:, at] & 0x0F) | (((d >> (4 * k)) & 0x0F) << 4).to(torch.uint8)
    else:
        for at in SCALE_AT[name]:
            raw[:, at] = (d & 0xFF).to(torch.uint8)
            raw[:, at + 1] = ((d >> 8) & 0xFF).to(torch.uint8)
    return raw.reshape(copies, -1)


def graph_us(torch, launch, G, reps=10):
    """launch(i) for i < G captured once in a graph on a side stream; the average microseconds a launch over `reps`
    replays, events recorded on that stream"""
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        for i in range(G):
            assert launch(i, s.cuda_stream) is not False, "a launch was refused"
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            for i in range(G):
                launch(i, s.cuda_stream)
    torch.cuda.synchronize()
    ev = Events(torch)
    with torch.cuda.stream(s):
        graph.replay()
        ms = ev.time(graph.replay, reps)
    return ms * 1e3 / (reps * G)


def gemv_extras(torch, capi, bs1_only=False):
    """configs 1 and 2: one matrix (rotated copies, more than 2 GiB) a launch - the fp32 matvec (mv_strided), the lane's
    int8 matvec (q8_group_tok, x rounded beforehand) and the f16 MFMA matmul (mm_run, x16 beforehand) at 8 / 64;
    bs1_only: one token alone (the metric's GEMV half on its own configs, in every run)"""
    L = capi.lib()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    out = {}
    for name, rows, cols, batches in (("Q4_0", 8192, 2048, (1,)), ("Q4_K", 6144, 2048, (1,) if bs1_only else (1, 8, 64)),
                                      ("Q3_K", 6144, 2048, (1,) if bs1_only else (1, 8, 64))):
        v, b = BLOCK[name]
        wbytes = rows * cols // v * b
        copies = max(2, math.ceil(2.2e9 / wbytes))
        W = blocks_of(torch, gen, name, rows, cols, copies)
        t = TYPE_ID[name]
        for n in batches:
            x = torch.randn(n, cols, device="cuda", generator=gen)
            y = torch.zeros(n, rows, device="cuda")
            G = min(copies, 64)
            us = graph_us(torch, lambda i, st: L.mv_strided(t, capi.addr(W[i]), rows, cols, capi.addr(x), cols, n,
                                                            capi.addr(y), rows, st), G)
            nb = wbytes + n * cols * 4 + n * rows * 4
            out["%s_%dx%d_mv_f32_bs%d" % (name, cols, rows, n)] = {"us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                                                  "contract": "mv fp32 (the reference's bits)"}
            if n <= 8:
                q = torch.zeros(n, cols, dtype=torch.int8, device="cuda")
                d = torch.zeros(n, cols // 32, device="cuda")
                assert L.q8_round(capi.addr(x), n, cols, cols, capi.addr(q), capi.addr(d), None)
                tabs = [torch.tensor([W[i].data_ptr()], dtype=torch.int64, device="cuda") for i in range(G)]
                cnt = torch.tensor([n], dtype=torch.int32, device="cuda")
                xrow = torch.zeros(1, dtype=torch.int32, device="cuda")
                us = graph_us(torch, lambda i, st: L.q8_group_tok(t, capi.addr(tabs[i]), capi.addr(cnt),
                                                                  capi.addr(xrow), None, 1, n, rows, cols, capi.addr(q),
                                                                  capi.addr(d), capi.addr(y), rows, st), G)
                nb = wbytes + n * (cols + cols // 32 * 4) + n * rows * 4
                out["%s_%dx%d_lane_int8_bs%d" % (name, cols, rows, n)] = {
                    "us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                    "contract": "lane int8, build-defined for %s (the reference's lane has no %s contract)" % (name, name)}
            if n >= 8:
                x16 = torch.zeros((n + 15) // 16 * 16 * cols, dtype=torch.float16, device="cuda")
                assert L.mm_x16(capi.addr(x), cols, n, cols, capi.addr(x16), None, None)
                us = graph_us(torch, lambda i, st: L.mm_run(t, capi.addr(W[i]), rows, cols, capi.addr(x16), n,
                                                            capi.addr(y), rows, st), G)
                nb = wbytes + n * cols * 2 + n * rows * 4
                out["%s_%dx%d_mm_f16_bs%d" % (name, cols, rows, n)] = {
                    "us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                    "TFLOP/s": round(2 * rows * cols * n / us / 1e6, 2),
                    "contract": "mm f16 (the reference's K split, within its bound)"}
        del W
        torch.cuda.empty_cache()
    return out


def deepseek_extras(torch, capi, steps=256):
    """config 4: the DeepSeek-style expert layer (hidden 7168, expert ff 2048, 256 routed experts top-8 plus the shared
    one as a ninth pick) through osmos_lane_layer, IQ1_S / IQ1_M / IQ2_XXS, batch 1 and 4"""
    from libosmos_amd.layer import LaneLayer
    dim, ff, n_exp, k = 7168, 2048, 257, 9
    gen = torch.Generator(device="cuda")
    gen.manual_seed(4)
    rng = torch.Generator(device="cpu")
    rng.manual_seed(5)
    out = {}
    for name in ("IQ1_S", "IQ1_M", "IQ2_XXS"):
        v, b = BLOCK[name]
        per_mat = ff * dim // v * b
        mats = [blocks_of(torch, gen, name, ff, dim, n_exp), blocks_of(torch, gen, name, ff, dim, n_exp),
                blocks_of(torch, gen, name, dim, ff, n_exp)]
        t = TYPE_ID[name]
        lay = LaneLayer(t, t, dim, ff, n_exp, k, *mats)
        for n in (1, 4):
            G = 64
            ids = torch.stack([torch.stack([torch.cat([torch.randperm(n_exp - 1, generator=rng)[:k - 1],
                                                       torch.tensor([n_exp - 1])]) for _ in range(n)])
                               for _ in range(G)]).to(torch.int32).cuda()
            w = torch.softmax(torch.randn(G, n, k, generator=rng), dim=-1).cuda()
            x = torch.randn(G, n, dim, generator=rng).cuda()
            add = torch.zeros(n, dim, device="cuda")
            y = torch.zeros(G, n, dim, device="cuda")
            lay.workspace(n)
            us = graph_us(torch, lambda i, st: lay.forward(x[i], ids[i], w[i], add, y[i], stream=st), G,
                          reps=max(1, steps // G))
            distinct = sum(len(set(ids[i].reshape(-1).tolist())) for i in range(G)) / G
            nb = distinct * 3 * per_mat + n * dim * 8
            out["deepseek_layer_%s_bs%d" % (name, n)] = {"us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                                         "MB_per_step": round(nb / 1e6, 2)}
        del lay, mats
        torch.cuda.empty_cache()
    return out


def engine_step_extras(torch, capi, copies=16):
    """config 3 at batch 1 through the reference engine's own call sequence (src/run/hip_lane.c: q8_gate_up with each
    expert's matrices in pointer tables, q8_round of h, q8_group_tok, ops_gather_sum_add), each launch graph-timed on
    rotated weight copies; the drop-in path for an engine that does not call osmos_lane_layer"""
    L = capi.lib()
    k, dim, ff = 10, 2048, 512
    gen = torch.Generator(device="cuda")
    gen.manual_seed(3)
    G = blocks_of(torch, gen, "IQ3_XXS", ff * k, dim, copies)
    U = blocks_of(torch, gen, "IQ3_XXS", ff * k, dim, copies)
    D = blocks_of(torch, gen, "IQ3_XXS", dim * k, ff, copies)
    gb, db = ff * (dim // 256) * 98, dim * (ff // 256) * 98
    tab = lambda M, b: [torch.tensor([M[c].data_ptr() + e * b for e in range(k)], dtype=torch.int64, device="cuda")  # noqa: E731
                        for c in range(copies)]
    tg, tu, td = tab(G, gb), tab(U, gb), tab(D, db)
    x = torch.randn(1, dim, device="cuda", generator=gen)
    q = torch.zeros(1, dim, dtype=torch.int8, device="cuda")
    d = torch.zeros(1, dim // 32, device="cuda")
    assert L.q8_round(capi.addr(x), 1, dim, dim, capi.addr(q), capi.addr(d), None)
    cnt = torch.ones(k, dtype=torch.int32, device="cuda")
    hrow = torch.arange(k, dtype=torch.int32, device="cuda")
    xin0 = torch.zeros(k, dtype=torch.int32, device="cuda")
    scale = torch.rand(k, device="cuda", generator=gen)
    h = torch.zeros(k, ff, device="cuda")
    hq = torch.zeros(k, ff, dtype=torch.int8, device="cuda")
    hd = torch.zeros(k, ff // 32, device="cuda")
    ye = torch.zeros(k, dim, device="cuda")
    y = torch.zeros(1, dim, device="cuda")
    add = torch.zeros(1, dim, device="cuda")
    order = torch.arange(k, dtype=torch.int32, device="cuda")
    us = {
        "q8_gate_up": graph_us(torch, lambda i, st: L.q8_gate_up(
            18, capi.addr(tg[i]), capi.addr(tu[i]), capi.addr(cnt), capi.addr(hrow), capi.addr(xin0), None, k, 1, ff,
            dim, capi.addr(q), capi.addr(d), capi.addr(scale), math.inf, capi.addr(h), ff, st), copies),
        "q8_round": graph_us(torch, lambda i, st: L.q8_round(capi.addr(h), k, ff, ff, capi.addr(hq), capi.addr(hd), st),
                             copies),
        "q8_group_tok": graph_us(torch, lambda i, st: L.q8_group_tok(
            18, capi.addr(td[i]), capi.addr(cnt), capi.addr(hrow), None, k, 1, dim, ff, capi.addr(hq), capi.addr(hd),
            capi.addr(ye), dim, st), copies),
        "ops_gather_sum_add": graph_us(torch, lambda i, st: L.ops_gather_sum_add(
            capi.addr(y), capi.addr(ye), capi.addr(order), k, 1, dim, capi.addr(add), st), copies),
    }
    total = sum(us.values())
    nbytes = k * (2 * gb + db) + dim * 5 + dim * 4
    return {"qwen_engine_step_iq3xxs_bs1": {"us": round(total, 2), "GB/s": round(nbytes / total / 1e3, 1),
                                             "launches_us": {n: round(v, 2) for n, v in us.items()}}}


SIMDS, CLOCK_GHZ = 1024, 2.4  # MI355X: 256 CUs x 4 SIMDs; a wave64 VALU instruction issues in 4 cycles of a SIMD


def contract_floor(outputs, groups, valu_per=4):
    """the bit-exact contract's own VALU floor: every (output, 32-value group) takes `valu_per` VALU operations that
    no reassociation may merge (mmq: the group's product, the dot's conversion and two fma; the lane: the two half
    products, their sum and the chain's fma), 64 lanes a wave instruction, 4 cycles each on one of 1024 SIMDs at
    2.4 GHz: returns (wave instructions, microseconds)"""
    winst = outputs * groups * valu_per / 64.0
    return winst, winst * 4 / (SIMDS * CLOCK_GHZ * 1e3)


def with_floor(entry, outputs, groups):
    winst, floor = contract_floor(outputs, groups)
    entry["contract_valu_winst_M"] = round(winst / 1e6, 1)
    entry["contract_floor_us"] = round(floor, 1)
    entry["frac_of_contract_floor"] = round(floor / entry["us"], 3)
    return entry


def roof_frac(us, nbytes, ops, peak_t):
    """the config's roofline time, max(bytes / HBM peak, ops / MFMA peak), over the measured time"""
    return round(max(nbytes / (HBM_PEAK_GBS * 1e3), ops / (peak_t * 1e6)) / us, 4)


def prefill_extras(torch, capi):
    """config 5: 512 tokens routed top-8 over 256 experts with Zipf(1.1) load, each expert's tokens gathered in whole
    tiles: Q4_K down (2048 -> 7168) on the int8 matrix cores (mmq_group, its x8 beforehand) and IQ2_XXS gate
    (7168 -> 2048) on the f16 ones (mm_group, its x16 beforehand) and on the int8 ones under the lane contract
    (osmos_lane_group, its q8 rows beforehand); TOPS / TFLOP/s and the fraction of MI355X's dense peaks (int8
    5.0 POPS, f16 2.5 PFLOP/s)"""
    import numpy as np
    L = capi.lib()
    n_tok, n_exp, k = 512, 256, 8
    rng = np.random.default_rng(11)
    p = 1.0 / np.arange(1, n_exp + 1) ** 1.1
    p /= p.sum()
    ids = np.stack([rng.choice(n_exp, k, replace=False, p=p) for _ in range(n_tok)])
    cnt = np.bincount(ids.reshape(-1), minlength=n_exp).astype(np.int32)
    pairs = [[] for _ in range(n_exp)]
    for t in range(n_tok):
        for e in ids[t]:
            pairs[e].append(t)
    soff = np.zeros(n_exp, np.uint32)
    idx = []
    for e in range(n_exp):
        soff[e] = len(idx)
        idx += pairs[e] + [-1] * ((-len(pairs[e])) % 16)
    slots = len(idx)
    idx_d = torch.tensor(idx, dtype=torch.int32, device="cuda")
    cnt_d = torch.tensor(cnt, device="cuda")
    gen = torch.Generator(device="cuda")
    gen.manual_seed(12)
    out = {"routing": {"tokens": n_tok, "experts": n_exp, "top_k": k, "zipf": 1.1, "busiest": int(cnt.max()),
                       "active_experts": int((cnt > 0).sum()), "slots": slots}}
    pairs_n = int(cnt.sum())
    # Q4_K down on int8 MFMA: rows 7168, cols 2048
    rows, cols = 7168, 2048
    W = blocks_of(torch, gen, "Q4_K", rows, cols, n_exp)
    wt = torch.tensor([W[e].data_ptr() for e in range(n_exp)], dtype=torch.int64, device="cuda")
    x = torch.randn(n_tok, cols, device="cuda", generator=gen)
    x8 = torch.zeros(slots * cols, dtype=torch.int8, device="cuda")
    dx = torch.zeros(slots * cols // 32, device="cuda")
    sx = torch.zeros(slots * cols // 32, device="cuda")
    assert L.mmq_x8_rows(capi.addr(x), cols, capi.addr(idx_d), slots, cols, capi.addr(x8), capi.addr(dx),
                         capi.addr(sx), None)
    soff_d = torch.tensor(soff, device="cuda")
    yoff_d = torch.tensor(soff.astype(np.int64) * rows, device="cuda").to(torch.int32)
    y = torch.zeros(slots * rows, device="cuda")
    us = graph_us(torch, lambda i, st: L.mmq_group(12, capi.addr(wt), capi.addr(cnt_d), n_exp, int(cnt.max()), rows,
                                                   cols, capi.addr(x8), capi.addr(dx), capi.addr(sx),
                                                   capi.addr(soff_d), capi.addr(y), capi.addr(yoff_d), rows, st), 4)
    tops = 2.0 * rows * cols * pairs_n / us / 1e6
    nbytes = int((cnt > 0).sum()) * rows * (cols // 256) * 144 + slots * cols * 9 // 8 + pairs_n * rows * 4
    out["prefill_q4k_down_mmq_int8"] = with_floor(
        {"us": round(us, 1), "TOPS": round(tops, 2), "pct_int8_mfma_peak": round(100 * tops / INT8_PEAK_TOPS, 3),
         "roofline_frac": roof_frac(us, nbytes, 2.0 * rows * cols * pairs_n, INT8_PEAK_TOPS)},
        pairs_n * rows, cols // 32)
    # the dense sub-shape: one Q4_K expert 2048 -> 7168 over all 512 tokens (32 full tiles: no padded slots) - the
    # compute-bound case of the same kernel
    idx1 = torch.arange(n_tok, dtype=torch.int32, device="cuda")
    x8d = torch.zeros(n_tok * cols, dtype=torch.int8, device="cuda")
    dxd = torch.zeros(n_tok * cols // 32, device="cuda")
    sxd = torch.zeros(n_tok * cols // 32, device="cuda")
    assert L.mmq_x8_rows(capi.addr(x), cols, capi.addr(idx1), n_tok, cols, capi.addr(x8d), capi.addr(dxd),
                         capi.addr(sxd), None)
    one = torch.tensor([n_tok], dtype=torch.int32, device="cuda")
    z = torch.zeros(1, dtype=torch.int32, device="cuda")
    yd = torch.zeros(n_tok * rows, device="cuda")
    us = graph_us(torch, lambda i, st: L.mmq_group(12, capi.addr(wt), capi.addr(one), 1, n_tok, rows, cols,
                                                   capi.addr(x8d), capi.addr(dxd), capi.addr(sxd), capi.addr(z),
                                                   capi.addr(yd), capi.addr(z), rows, st), 8)
    tops = 2.0 * rows * cols * n_tok / us / 1e6
    out["dense_q4k_down_mmq_int8_512tok"] = with_floor({
        "us": round(us, 2), "TOPS": round(tops, 2), "pct_int8_mfma_peak": round(100 * tops / INT8_PEAK_TOPS, 3),
        "roofline_frac": roof_frac(us, rows * (cols // 256) * 144 + n_tok * cols * 9 // 8 + n_tok * rows * 4,
                                   2.0 * rows * cols * n_tok, INT8_PEAK_TOPS)}, n_tok * rows, cols // 32)
    del W, wt, x8, dx, sx, y, x8d, dxd, sxd, yd
    torch.cuda.empty_cache()
    # IQ2_XXS gate on f16 MFMA: rows 2048, cols 7168
    rows, cols = 2048, 7168
    W = blocks_of(torch, gen, "IQ2_XXS", rows, cols, n_exp)
    wt = torch.tensor([W[e].data_ptr() for e in range(n_exp)], dtype=torch.int64, device="cuda")
    x = torch.randn(n_tok, cols, device="cuda", generator=gen)
    x16 = torch.zeros(slots * cols, dtype=torch.float16, device="cuda")
    assert L.mm_x16_rows(capi.addr(x), cols, capi.addr(idx_d), slots, cols, capi.addr(x16), None, None)
    xoff_d = torch.tensor(soff.astype(np.int64) * cols, device="cuda").to(torch.int32)
    yoff_d = torch.tensor(soff.astype(np.int64) * rows, device="cuda").to(torch.int32)
    y = torch.zeros(slots * rows, device="cuda")
    us = graph_us(torch, lambda i, st: L.mm_group(16, capi.addr(wt), capi.addr(cnt_d), n_exp, int(cnt.max()), rows,
                                                  cols, capi.addr(x16), capi.addr(xoff_d), cols, capi.addr(y),
                                                  capi.addr(yoff_d), rows, st), 4)
    tf = 2.0 * rows * cols * pairs_n / us / 1e6
    wbytes = int((cnt > 0).sum()) * rows * (cols // 256) * 66
    out["prefill_iq2xxs_gate_mm_f16"] = {"us": round(us, 1), "TFLOP/s": round(tf, 2),
                                         "pct_f16_mfma_peak": round(100 * tf / F16_PEAK_TFLOPS, 3),
                                         "roofline_frac": roof_frac(us, wbytes + slots * cols * 2 + pairs_n * rows * 4,
                                                                    2.0 * rows * cols * pairs_n, F16_PEAK_TFLOPS)}
    # the same gate on the int8 matrix cores under the lane contract (the reference CPU lane's bits): each expert's
    # tokens gathered in order, rounded (q8_round), then osmos_lane_group
    order = [t for e in range(n_exp) for t in pairs[e]]
    xg = x[torch.tensor(order, device="cuda")].contiguous()
    q8 = torch.zeros(pairs_n, cols, dtype=torch.int8, device="cuda")
    d8 = torch.zeros(pairs_n, cols // 32, device="cuda")
    assert L.q8_round(capi.addr(xg), pairs_n, cols, cols, capi.addr(q8), capi.addr(d8), None)
    xrow = torch.tensor(np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(np.int32), device="cuda")
    y = torch.zeros(pairs_n, rows, device="cuda")
    us = graph_us(torch, lambda i, st: L.osmos_lane_group(16, capi.addr(wt), capi.addr(cnt_d), capi.addr(xrow), n_exp,
                                                          int(cnt.max()), rows, cols, capi.addr(q8), capi.addr(d8),
                                                          capi.addr(y), rows, st), 4)
    tops = 2.0 * rows * cols * pairs_n / us / 1e6
    out["prefill_iq2xxs_gate_lane_int8"] = with_floor(
        {"us": round(us, 1), "TOPS": round(tops, 2), "pct_int8_mfma_peak": round(100 * tops / INT8_PEAK_TOPS, 3),
         "roofline_frac": roof_frac(us, wbytes + pairs_n * cols * 9 // 8 + pairs_n * rows * 4,
                                    2.0 * rows * cols * pairs_n, INT8_PEAK_TOPS)},
        pairs_n * rows, cols // 32)
    del W, wt, x16, y
    torch.cuda.empty_cache()
    return out


def moe_layer_bench(torch, capi, n_tok, steps, warmup, rotate_bytes=2.2e9, seed=0):
    """config 3: returns a dict of the step's timing and bytes"""
    from libosmos_amd.layer import LaneLayer
    T = 18  # IQ3_XXS
    dim, ff, n_exp, k = 2048, 512, 512, 10
    per_expert = 3 * (ff * (dim // 256) * 98)  # gate + up + down: 1,204,224 B
    n_layers = max(2, math.ceil(rotate_bytes / (per_expert * n_exp)))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    layers = []
    for _ in range(n_layers):
        mats = [iq_weights(torch, gen, n_exp * ff * dim // 256, 98).reshape(n_exp, -1) for _ in range(2)]
        mats.append(iq_weights(torch, gen, n_exp * dim * ff // 256, 98).reshape(n_exp, -1))
        layers.append(LaneLayer(T, T, dim, ff, n_exp, k, *mats))
    G = 64  # steps a graph
    rng = torch.Generator(device="cpu")
    rng.manual_seed(seed + 1)
    ids = torch.stack([torch.stack([torch.randperm(n_exp, generator=rng)[:k] for _ in range(n_tok)]) for _ in range(G)])
    ids = ids.to(torch.int32).cuda()
    w = torch.softmax(torch.randn(G, n_tok, k, generator=rng), dim=-1).cuda()
    x = torch.randn(G, n_tok, dim, generator=rng).cuda()
    add = torch.zeros(n_tok, dim, device="cuda")
    out = torch.zeros(G, n_tok, dim, device="cuda")
    for L in layers:
        L.workspace(n_tok)
    # algorithmic bytes a step: each distinct expert's three matrices once, x read, the output written
    distinct = [len(set(ids[s].reshape(-1).tolist())) for s in range(G)]
    step_bytes = sum(distinct) / G * per_expert + n_tok * dim * 4 * 2 + n_tok * k * 8

    s = torch.cuda.Stream()

    def run(st):
        layers[st % n_layers].forward(x[st % G], ids[st % G], w[st % G], add, out[st % G], stream=s.cuda_stream)

    # exactly `warmup` untimed steps: the first eager (the first use of every code path), the rest as one captured
    # graph - a process's first graph launch pays a one-time cost of the runtime (20 timed steps: 12.1 us a step when
    # the timed graph is the process's first, 11.3 when it is not), which belongs to the warmup, not to the steps
    with torch.cuda.stream(s):
        for st in range(min(warmup, 1)):
            run(st)
    torch.cuda.synchronize()
    if warmup > 1:
        wg = torch.cuda.CUDAGraph()
        with torch.cuda.stream(s):
            with torch.cuda.graph(wg, stream=s):
                for st in range(1, warmup):
                    run(st)
        torch.cuda.synchronize()
        wg.replay()
        torch.cuda.synchronize()
        del wg
    # the timed steps: exactly `steps`, as replays of a graph of min(steps, G) steps plus one graph of the remainder
    per = min(steps, G)
    graphs = []
    for n in ([per] * (steps // per)) + ([steps % per] if steps % per else []):
        if not graphs or n != per:
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.stream(s):
                with torch.cuda.graph(graph, stream=s):
                    for st in range(n):  # (steps after the warmup's: no timed step repeats a warmup step's experts)
                        run(warmup + st)
            graphs.append((graph, n))
        else:
            graphs.append(graphs[0])
    torch.cuda.synchronize()
    ev = Events(torch)
    ms = ev.time(lambda: [g.replay() for g, _ in graphs], 1)
    n_steps = sum(n for _, n in graphs)
    assert n_steps == steps
    ms_step = ms / n_steps
    return dict(n_tok=n_tok, steps=n_steps, ms_per_step=ms_step, step_bytes=step_bytes,
                gbs=step_bytes / (ms_step * 1e-3) / 1e9, layers=layers, ids=ids, w=w, x=x, G=G, n_layers=n_layers,
                dims=(dim, ff, n_exp, k), per_expert=per_expert)


def half_bench(torch, capi, lay, half, reps=20):
    """one fused kernel of the layer alone: osmos_lane_gate_up (fused::gu1_kernel at one token) or osmos_lane_down (fused::dn_kernel)
    over the timed steps' routing and rotated weights, G launches back to back in a graph on stream s; the average
    duration a launch from events recorded on s; its algorithmic bytes (each distinct expert's matrices once, the
    activations in, the outputs out)"""
    dim, ff, n_exp, k = lay["dims"]
    layers, ids, w, x, G, n_layers = lay["layers"], lay["ids"], lay["w"], lay["x"], lay["G"], lay["n_layers"]
    n_tok = lay["n_tok"]
    L = capi.lib()
    h = torch.randn(G, n_tok * k, ff, device="cuda")
    add = torch.zeros(n_tok, dim, device="cuda")
    out = torch.zeros(G, n_tok, dim, device="cuda")
    s = torch.cuda.Stream()

    def launch_all():
        for st in range(G):
            d = ctypes.byref(layers[st % n_layers].desc)
            if half == "gate_up":
                ok = L.osmos_lane_gate_up(d, capi.addr(x[st]), n_tok, capi.addr(ids[st]), capi.addr(w[st]),
                                          capi.addr(h[st]), s.cuda_stream)
            else:
                ok = L.osmos_lane_down(d, capi.addr(h[st]), n_tok, capi.addr(ids[st]), capi.addr(add),
                                       capi.addr(out[st]), s.cuda_stream)
            assert ok

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        launch_all()
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=s):
            launch_all()
    torch.cuda.synchronize()
    ev = Events(torch)
    with torch.cuda.stream(s):
        graph.replay()
        ms = ev.time(graph.replay, reps)
    us = ms * 1e3 / (reps * G)
    distinct = sum(len(set(ids[st].reshape(-1).tolist())) for st in range(G)) / G
    per_mat = ff * (dim // 256) * 98
    if half == "gate_up":
        nbytes = distinct * 2 * per_mat + n_tok * dim * 4 + n_tok * k * 8 + n_tok * k * ff * 4
    else:
        nbytes = distinct * per_mat + n_tok * k * ff * 4 + n_tok * k * 4 + 2 * n_tok * dim * 4
    return dict(us=us, bytes=nbytes, gbs=nbytes / (us * 1e-6) / 1e9)


def llc_bytes():
    """the host's last-level cache in bytes, summed over the distinct caches the process's CPUs share (sysfs); 0 if
    unknown"""
    seen, total = set(), 0
    for c in sorted(os.sched_getaffinity(0)):
        base = "/sys/devices/system/cpu/cpu%d/cache" % c
        try:
            idx = max((int(d[5:]) for d in os.listdir(base) if d.startswith("index")), default=None)
            if idx is None:
                continue
            with open("%s/index%d/shared_cpu_list" % (base, idx)) as f:
                key = (idx, f.read().strip())
            if key in seen:
                continue
            seen.add(key)
            with open("%s/index%d/size" % (base, idx)) as f:
                v = f.read().strip()
            total += int(v[:-1]) * {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}[v[-1]] if v[-1] in "KMG" else int(v)
        except (OSError, ValueError):
            continue
    return total


def cpu_baseline(lay, seconds=10.0):
    """the reference's CPU path on this host's cores for one step of the same layer (bs as the GPU's), a bounded
    sample: repetitions of the layer until ~`seconds` of CPU time, cold: the repetitions rotate through copies of the
    step's expert weights (the same bytes at other addresses) totalling at least four times the host's last-level
    cache, so each step reads its weights from DRAM as a decode step does"""
    import numpy as np
    from oracle import orc
    torch = __import__("torch")
    dim, ff, n_exp, k = lay["dims"]
    n_tok = lay["n_tok"]
    R = orc.ref()
    kind = "reference"
    if R is None or not R.ref_q8_ready():
        kind = "port"
    ids = lay["ids"][0].cpu().numpy()
    lyr = lay["layers"][0]
    experts = sorted(set(ids.reshape(-1).tolist()))
    mats = {}
    for nm, t in zip(("g", "u", "d"), lyr.tensors):
        mats[nm] = [t[e].cpu().numpy() for e in experts]
    step_bytes = len(experts) * lay["per_expert"] + n_tok * dim * 8
    llc = llc_bytes()
    copies = max(4, -(-4 * max(llc, 256 << 20) // max(step_bytes, 1)))
    copies = min(copies, max(1, int(4e9 // step_bytes)))
    rot = {nm: [np.copy(m) for _ in range(copies) for m in ms] for nm, ms in mats.items()}
    pairs = sorted((int(ids[t, j]), t * k + j) for t in range(n_tok) for j in range(k))
    r0 = np.array([min(r for r, (e, _) in enumerate(pairs) if e == ex) for ex in experts], np.uint32)
    cnt = np.array([sum(1 for e, _ in pairs if e == ex) for ex in experts], np.uint32)
    x = lay["x"][0].cpu().numpy()
    rows_x = np.stack([x[m // k] for _, m in pairs]).astype(np.float32)
    scale = lay["w"][0].cpu().numpy().reshape(-1)[[m for _, m in pairs]].astype(np.float32)
    P = ctypes.c_void_p
    tab = lambda ms: (P * len(ms))(*[m.ctypes.data for m in ms])  # noqa: E731
    threads = len(os.sched_getaffinity(0))
    y = np.zeros((len(pairs), dim), np.float32)
    if kind == "reference":
        q, d = orc.q8_round(rows_x, R)
        tg, tu, td = tab(rot["g"]), tab(rot["u"]), tab(rot["d"])

        def run(th, reps):
            assert R.ref_lane_layer_rot(18, dim, ff, tg, tu, td, orc.ptr(r0), orc.ptr(cnt), len(experts), len(pairs),
                                        orc.ptr(q), orc.ptr(d), orc.ptr(scale), orc.ptr(y), th, reps, copies)
            return

        run(threads, copies)  # warm-up: one pass over every copy (page faults, thread start)
        t0 = time.perf_counter()
        run(threads, 10)
        per = (time.perf_counter() - t0) / 10
        reps = max(copies, int(seconds / max(per, 1e-6)))
        t0 = time.perf_counter()
        run(threads, reps)
        per = (time.perf_counter() - t0) / reps
        # one core as well (the same layer, a quarter of the sample's time)
        t0 = time.perf_counter()
        run(1, 1)
        per1 = time.perf_counter() - t0
        reps1 = max(2, int(seconds / 4 / max(per1, 1e-6)))
        t0 = time.perf_counter()
        run(1, reps1)
        per1 = (time.perf_counter() - t0) / reps1
    else:
        threads = 1
        t0 = time.perf_counter()
        reps = 0
        while time.perf_counter() - t0 < seconds:
            c = reps % copies
            sl = slice(c * len(experts), (c + 1) * len(experts))
            assert orc.orc().orc_lane_layer(18, 18, dim, ff, math.inf, orc.ptr(rows_x), orc.ptr(scale), len(pairs),
                                            tab(rot["g"][sl]), tab(rot["u"][sl]), tab(rot["d"][sl]), orc.ptr(r0),
                                            orc.ptr(cnt), len(experts), orc.ptr(y))
            reps += 1
        per = (time.perf_counter() - t0) / reps
    del torch, rot
    cold = "cold: %d weight copies rotated (%.0f MB against a %.0f MB last-level cache)" % (
        copies, copies * step_bytes / 1e6, llc / 1e6)
    out = {"value": round(step_bytes / per / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": kind,
           "sample": "%d x one %d-token step of the same layer (%d experts' gate/up/down, int8 lane), %.2f ms a step; %s"
                     % (reps, n_tok, len(experts), per * 1e3, cold),
           "llc_bytes": llc}
    if kind == "reference":
        out["one_core"] = {"value": round(step_bytes / per1 / 1e9, 3), "unit": "GB/s",
                           "sample": "%d x the same step on one thread, %.2f ms a step (the same rotation)"
                                     % (reps1, per1 * 1e3)}
    return out


def ceilings(torch):
    """the box's own ceilings for the roofline: a best-shaped streaming read (bench-calibration kernel calib_read: every
    thread a run of 16-byte loads all in flight) of the layer kernels' byte counts and of large reads, each launch on
    fresh bytes of a 4 GiB pool (beyond the 256 MB Infinity Cache), graph-launched like the bench; and chains of dense
    MFMAs (int8 and f16) over 2048 workgroups: the matrix cores' measured peak"""
    L = ctypes.CDLL(os.path.join(ROOT, "libosmos_amd", "libosmos_calib.so"))
    L.calib_read.restype = ctypes.c_bool
    L.calib_read.argtypes = [ctypes.c_void_p, ctypes.c_uint64] + [ctypes.c_uint32] * 3 + [ctypes.c_void_p] * 2
    L.calib_mfma.restype = ctypes.c_bool
    L.calib_mfma.argtypes = [ctypes.c_uint32] * 3 + [ctypes.c_void_p] * 2
    pool_bytes = 4 << 30
    pool = torch.empty(pool_bytes, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(1 << 16, dtype=torch.int32, device="cuda")
    out = {"read": {}, "mfma": {}}
    for nbytes in (4050944, 8056832, 12107776, 64 << 20, 1 << 30):
        best = None
        for threads, unroll in ((256, 4), (256, 8), (256, 16), (512, 8), (1024, 4), (1024, 8)):
            for grid in (256, 512, 1024, 2048):
                if grid * threads * unroll * 16 > nbytes * 2:
                    continue
                slots = max(1, pool_bytes // nbytes)
                G = min(32, slots)

                def launch(i, st, threads=threads, unroll=unroll, grid=grid):
                    src = pool.data_ptr() + (i % slots) * (nbytes // 4096 * 4096)
                    return L.calib_read(src, nbytes, grid, threads, unroll, sink.data_ptr(), st)
                us = graph_us(torch, launch, G, reps=5)
                if best is None or us < best[0]:
                    best = (us, threads, unroll, grid)
        us, threads, unroll, grid = best
        out["read"][str(nbytes)] = {"us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                                    "pct_hbm_peak": round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 1),
                                    "threads": threads, "unroll": unroll, "workgroups": grid}
        log("read %d B: %.2f us (%d threads x %d, %d workgroups)" % (nbytes, us, threads, unroll, grid))
    # the routed layer's pattern: 20 regions of 401,408 bytes (10 experts' gate and up, IQ3_XXS 512 x 2048) picked per
    # launch through a device array of region indices from the pool
    L.calib_gather.restype = ctypes.c_bool
    L.calib_gather.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint32,
                               ctypes.c_uint32, ctypes.c_void_p, ctypes.c_void_p]
    region, n_reg = 401408, 20
    gen = torch.Generator(device="cpu")
    gen.manual_seed(7)
    n_slots = pool_bytes // region
    id_sets = [torch.randperm(n_slots, generator=gen)[:n_reg].to(torch.int32).cuda() for _ in range(32)]
    best = None
    for threads, unroll in ((64, 4), (128, 4), (256, 1), (256, 2), (256, 4), (256, 8), (512, 4)):
        us = graph_us(torch, lambda i, st, threads=threads, unroll=unroll: L.calib_gather(
            pool.data_ptr(), id_sets[i].data_ptr(), n_reg, region, threads, unroll, sink.data_ptr(), st), 32, reps=5)
        if best is None or us < best[0]:
            best = (us, threads, unroll)
    us, threads, unroll = best
    nb = region * n_reg
    out["read"]["gather_20x401408"] = {"us": round(us, 3), "GB/s": round(nb / us / 1e3, 1),
                                       "pct_hbm_peak": round(100 * nb / us / 1e3 / HBM_PEAK_GBS, 1),
                                       "threads": threads, "unroll": unroll}
    log("gather 20 x 401408 B through device ids: %.2f us (%d threads x %d)" % (us, threads, unroll))
    empty = graph_us(torch, lambda i, st: L.calib_read(pool.data_ptr(), 16, 1, 256, 4, sink.data_ptr(), st), 32)
    out["read"]["one_line_launch_us"] = round(empty, 3)
    blocks, iters = 2048, 4000
    for kind, name, mnk, peak in ((0, "int8_16x16x64", 16 * 16 * 64, INT8_PEAK_TOPS),
                                  (1, "int8_32x32x32", 32 * 32 * 32, INT8_PEAK_TOPS),
                                  (2, "f16_16x16x32", 16 * 16 * 32, F16_PEAK_TFLOPS),
                                  (3, "f16_32x32x16", 32 * 32 * 16, F16_PEAK_TFLOPS)):
        us = graph_us(torch, lambda i, st: L.calib_mfma(kind, blocks, iters, sink.data_ptr(), st), 4, reps=3)
        t = 2.0 * mnk * blocks * 4 * iters * 4 / us / 1e6
        out["mfma"][name] = {"us": round(us, 1), "T_per_s": round(t, 1), "pct_peak": round(100 * t / peak, 1)}
        log("mfma %s: %.1f T/s (%.1f %% of %g)" % (name, t, 100 * t / peak, peak))
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1280)
    ap.add_argument("--warmup", type=int, default=128)
    ap.add_argument("--all", action="store_true", help="also the other BASELINE configs, as extra lines")
    ap.add_argument("--only", default="3,12,4,5", help="with --all: which extras (3: bs 4/32, 12: configs 1-2, 4, 5)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run a plain device copy of 64 MiB, 8 times (the calibration kernel of a counter run)")
    ap.add_argument("--ceilings", action="store_true",
                    help="only the box's ceilings (streaming read, MFMA chains), one JSON line")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one MI355X: this build has no multi-GPU path (--gpus %d refused)" % args.gpus)
        sys.exit(2)
    import torch
    from libosmos_amd import capi
    capi.lib()
    torch.cuda.set_device(0)
    if args.ceilings:
        print(json.dumps({"ceilings": ceilings(torch)}))
        return
    log("config 3 layer, batch 1")
    lay = moe_layer_bench(torch, capi, 1, args.steps, args.warmup)
    log("  %.2f us a step, %.1f GB/s" % (lay["ms_per_step"] * 1e3, lay["gbs"]))
    ker = half_bench(torch, capi, lay, "gate_up")
    log("  gate/up kernel: %.2f us, %.1f GB/s" % (ker["us"], ker["gbs"]))
    dn = half_bench(torch, capi, lay, "down")
    log("  down kernel: %.2f us, %.1f GB/s" % (dn["us"], dn["gbs"]))
    line = {
        "metric": METRIC, "value": round(lay["gbs"], 2), "unit": "GB/s", "n_gpus": 1, "steps": lay["steps"],
        "warmup": args.warmup, "ms_per_step": round(lay["ms_per_step"], 6), "higher_is_better": True,
        "scaling": "weak", "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "qwen_moe_layer_iq3xxs_bs1", "hidden": 2048, "experts": 512, "expert_ff": 512,
                   "top_k": 10, "batch": 1, "weights": "IQ3_XXS", "contract": "lane int8 (bit-exact)",
                   "pct_hbm_peak": round(100 * lay["gbs"] / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(ker["gbs"], 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(ker["gbs"] / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "osm::fused::gu1_kernel<IQ3_XXS,1>", "us_per_launch": round(ker["us"], 3),
                     "bytes_per_launch": int(ker["bytes"])},
        "kernels": {"osm::fused::dn_kernel<IQ3_XXS,16,1>": {"us_per_launch": round(dn["us"], 3),
                                                          "bytes_per_launch": int(dn["bytes"]),
                                                          "GB/s": round(dn["gbs"], 2)}},
    }
    traffic = os.path.join(ROOT, "profiles", "gu1_kernel_iq3xxs_bs1_traffic.json")
    if os.path.exists(traffic):  # HBM bytes a launch, from the counter runs that file records
        with open(traffic) as f:
            line["roofline"]["traffic"] = json.load(f)["hbm_bytes_per_launch"]
    if args.copy_probe:
        a = torch.empty(64 << 20, dtype=torch.uint8, device="cuda")
        b = torch.empty_like(a)
        for _ in range(8):
            b.copy_(a)
        torch.cuda.synchronize()
    if not args.no_cpu:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(lay, args.cpu_seconds)
    # the metric's second half (batch-512 expert GEMM, int8 TOPS): config 5, in every run
    log("config 5 (the metric's batch-512 half)")
    del lay
    torch.cuda.empty_cache()
    prefill = prefill_extras(torch, capi)
    line["prefill_bs512"] = prefill
    # the metric's GEMV half on configs 1 and 2 (one token, HBM GB/s), in every run
    log("configs 1, 2 at one token")
    torch.cuda.empty_cache()
    gemv = gemv_extras(torch, capi, bs1_only=True)
    for v in gemv.values():
        v["pct_hbm_peak"] = round(100 * v["GB/s"] / HBM_PEAK_GBS, 2)
    line["gemv_bs1"] = gemv
    if args.all:
        torch.cuda.empty_cache()
        extra = {}
        only = set(args.only.split(","))
        if "3" in only:
            extra.update(engine_step_extras(torch, capi))
            torch.cuda.empty_cache()
        for n_tok in (4, 32) if "3" in only else ():
            lb = moe_layer_bench(torch, capi, n_tok, max(args.steps // 4, 64), 16)
            extra["qwen_moe_layer_iq3xxs_bs%d" % n_tok] = {"GB/s": round(lb["gbs"], 2),
                                                           "us_per_step": round(lb["ms_per_step"] * 1e3, 3)}
            del lb
            torch.cuda.empty_cache()
        if "12" in only:
            log("configs 1, 2")
            torch.cuda.empty_cache()
            extra.update(gemv_extras(torch, capi))
        if "4" in only:
            log("config 4")
            extra.update(deepseek_extras(torch, capi))
        if "5" in only:
            extra.update(prefill)
        line["extra"] = extra
    print(json.dumps(line))


if __name__ == "__main__":
    main()
