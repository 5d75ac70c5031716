#!/usr/bin/env python3
"""Benchmark of llm_mojo's quantized matmul path on one MI355X.

Metric: decode tok/s of GPT-2 124M int4-g32-a16 at batch 1
(config 0: seeded random-init weights, int8 per-channel head, int8 KV cache,
a 12-token random prompt, then 100 greedy tokens), plus the achieved HBM
bandwidth of the W4A16 group-32 GEMV at 4096 x 11008 against the 8 TB/s peak.

A step is one generation: the 12-token prompt forward and 100 greedy tokens,
each fed back on the device.  `value` follows the reference's tok/s
definition (gpt2t.mojo:968-1005): generated tokens over the decode span (99
decode forwards and 100 argmaxes), summed over the K timed steps; the
prompt's time is reported separately.  Weights, KV cache and activations are
resident in HBM before the timed region starts.

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Prints one JSON line on stdout; progress goes to stderr.
"""
import argparse
import json
import os
import subprocess
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

HBM_PEAK_GBS = 8000.0
PROMPT, GEN, SEED = 12, 100, 1337


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def graph_us(torch, ctx, stream, fn, n, replays=3):
    """Device time per launch of fn(0) .. fn(n - 1): the n launches captured
    once into a HIP graph and replayed, timed with HIP events on `stream`, so
    the host's enqueue rate (a ctypes call per launch from Python) cannot set
    the rate of short kernels.  fn must issue its work on ctx's stream."""
    with torch.cuda.stream(stream):
        ctx.set_stream(stream)
        for i in range(n):  # first launches (lazy set-up) outside the capture
            fn(i)
        stream.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
            for i in range(n):
                fn(i)
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(replays):
            g.replay()
        e1.record(stream)
        e1.synchronize()
        del g
    return e0.elapsed_time(e1) * 1000.0 / (replays * n)


def read_floor(torch, lm, ctx, stream, nbytes, nbuf, grid=2048, reps=None, graph=False):
    """Average duration of a pure read of nbytes (llmq_debug_read: 128-bit
    loads, no arithmetic) over nbuf distinct buffers, on `stream`; with
    graph, each launch's device time (graph_us), else HIP events over
    back-to-back launches from the host."""
    bufs = [torch.empty(nbytes // 16 * 16, dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
    out = torch.zeros(grid, dtype=torch.int32, device="cuda")
    reps = reps or max(60, 4 * nbuf)
    if graph:  # (at least 64 launches a graph: a replay's own start-up is then a small share)
        us = graph_us(torch, ctx, stream, lambda i: lm.debug_read(ctx, bufs[i % nbuf], out, grid),
                      max(nbuf, 64, min(reps, 4 * nbuf)))
        del bufs
        return us
    for i in range(2 * nbuf):
        lm.debug_read(ctx, bufs[i % nbuf], out, grid)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(reps):
        lm.debug_read(ctx, bufs[i % nbuf], out, grid)
    e1.record(stream)
    e1.synchronize()
    del bufs
    return e0.elapsed_time(e1) * 1000.0 / reps


READ_SWEEP_MB = [4, 8, 16, 26.82368, 64, 128, 256, 512, 1024]
READ_GRIDS = [256, 1024, 2048, 4096]


def read_sweep(torch, lm, ctx, rot_bytes=1 << 30):
    """What one launch of a pure read of n bytes takes from HBM on this box,
    n from 4 MB to 1 GiB (26.82 MB: the roofline GEMV's bytes), each over
    distinct buffers totalling >= 1 GiB (beyond the 256 MB Infinity Cache),
    best of four grid sizes, device time per launch (graph replay); and
    hipMemcpyAsync device-to-device of the same 26.82 MB (read + write)."""
    stream = torch.cuda.Stream()
    res = {}
    for mb in READ_SWEEP_MB:
        nbytes = int(mb * 1e6) // 16 * 16
        nbuf = max(2, -(-rot_bytes // nbytes))
        best = None
        for grid in READ_GRIDS:
            us = read_floor(torch, lm, ctx, stream, nbytes, nbuf, grid=grid, graph=True)
            if best is None or us < best[0]:
                best = (us, grid)
        res[f"{mb:g}MB"] = {"bytes": nbytes, "us": round(best[0], 3), "gbs": round(nbytes / best[0] / 1e3, 1),
                            "frac": round(nbytes / best[0] / 1e3 / HBM_PEAK_GBS, 4), "grid": best[1]}
        log("read sweep", mb, res[f"{mb:g}MB"])
    nbytes = int(26.82368e6) // 16 * 16
    nbuf = max(2, -(-rot_bytes // nbytes))
    src = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
    dst = [torch.empty(nbytes, dtype=torch.uint8, device="cuda") for _ in range(nbuf)]
    us = graph_us(torch, ctx, stream, lambda i: dst[i % nbuf].copy_(src[i % nbuf]), 2 * nbuf)
    res["memcpy_d2d_26.82MB"] = {"bytes_read": nbytes, "us": round(us, 3),
                                 "read_plus_write_gbs": round(2 * nbytes / us / 1e3, 1)}
    del src, dst
    ctx.set_stream(None)
    return res


def gemv_roofline(torch, lm, ctx, K=4096, N=11008, nbuf=36, reps=144):
    """The W4A16 g32 GEMV over `nbuf` distinct weight buffers (> 768 MiB in
    total, beyond the 256 MB Infinity Cache): `reps` launches rotating over
    them captured into a HIP graph and replayed, timed with HIP events on the
    stream they run on (graph_us), so the host's enqueue rate cannot set the
    rate.  The timed kernel is the GEMV proper over the token's
    prepared int16 activations (llmq_linear_act; llmq_act_prepare runs once
    before, as linear_team's thread 0 quantizes once per token), so its
    algorithmic bytes are nbytes(W) + 2K (int16 activations) + 4N (f32
    outputs).  Also reported: the float-input path (llmq_linear, the
    activation prologue in every workgroup) and the read floor, a pure read
    of the same bytes over as many buffers timed the same way."""
    stream = torch.cuda.Stream()
    mats = []
    with torch.cuda.stream(stream):
        ctx.set_stream(stream)
        g = torch.Generator(device="cuda").manual_seed(2002)
        for i in range(nbuf):
            src = torch.randn((K, N), device="cuda", generator=g) * 0.02
            mats.append(lm.HipQuantMatrix.from_f32(ctx, src, 4, 32, False, True))
            del src
        x = torch.randn((1, K), device="cuda", generator=g)
        out = torch.empty((1, N), device="cuda")
        act = torch.zeros(lm.act_bytes(K), dtype=torch.uint8, device="cuda")
        lm.act_prepare(ctx, x, act)

        us = graph_us(torch, ctx, stream, lambda i: lm.linear_act(ctx, out, act, mats[i % nbuf]), reps)
        us_float = graph_us(torch, ctx, stream, lambda i: lm.linear(ctx, out, x, mats[i % nbuf]), reps)
        wbytes = mats[0].nbytes()
        for m in mats:
            m.free()
        floor_us = read_floor(torch, lm, ctx, stream, wbytes, nbuf, reps=reps, graph=True)
    ctx.set_stream(None)
    alg = wbytes + 2 * K + 4 * N  # nbytes + int16 activations + f32 outputs
    return {"kernel": f"gemv_blk_kernel (W4A16 int4-g32, BLOCKED) {K}x{N}, prepared activations", "us": us,
            "alg_bytes": alg, "weight_bytes": wbytes, "buffers": nbuf, "gbs": alg / us / 1e3,
            "float_input_us": round(us_float, 2),
            "read_floor_us": round(floor_us, 2), "read_floor_gbs": round(wbytes / floor_us / 1e3, 1),
            "frac_of_read_floor": round(floor_us / us, 3)}


def measured_traffic():
    """HBM bytes per launch of the roofline GEMV from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE passes (profiles/), scaled by what the
    same counters read for a 1 GiB copy, and the kernel trace's average
    duration of the same command; (None, None) if absent."""
    p = os.path.join(HERE, "profiles", "gemv_a16_int4_g32_4096x11008.traffic.json")
    try:
        with open(p) as f:
            d = json.load(f)
        return d["traffic_bytes_per_launch"], d.get("kernel_trace_avg_us")
    except (OSError, KeyError, ValueError):
        return None, None


def copy_bandwidth(torch, nbytes=1 << 30, reps=20):
    """Device-to-device copy bandwidth (read + write bytes), for scale."""
    a = torch.empty(nbytes // 4, device="cuda")
    b = torch.empty_like(a)
    b.copy_(a)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        b.copy_(a)
    e1.record()
    e1.synchronize()
    return 2 * nbytes * reps / (e0.elapsed_time(e1) / 1000.0) / 1e9


GPT2_SHAPES = [("qkv", 768, 2304), ("proj", 768, 768), ("fc", 768, 3072), ("fcproj", 3072, 768)]
GEMV_FORMATS = [(4, 32), (4, 64), (4, 128), (8, 32), (8, 64), (8, 128)]


def gemv_micro(torch, lm, ctx, reps=200, rot_bytes=320 << 20):
    """Config 1: the one-token A16 GEMV at the GPT-2 shapes, int4 and int8 at
    groups 32 / 64 / 128, and the int8 per-channel head (768 x 50257), two
    ways: one matrix launched back to back (it stays in the 256 MB Infinity
    Cache, as in decode: `llc`), and over distinct copies totalling > 320 MiB
    (`hbm`, more than the 256 MB cache).  GB/s of nbytes + 2K + 4N per
    launch; each is set beside a pure read of the same bytes the same way
    (`*_floor_us`: the memory system's time for those bytes in one launch,
    LLC-resident or rotated).  Every time is device time per launch from a
    replayed HIP graph of the launches (graph_us): launched from Python one
    by one, these 3-10 us kernels would be timed at the host's enqueue rate."""
    stream = torch.cuda.Stream()
    res = {}
    with torch.cuda.stream(stream):
        ctx.set_stream(stream)
        g = torch.Generator(device="cuda").manual_seed(1001)
        cases = [(f"int{b}-g{gr} {n}", K, N, b, gr) for b, gr in GEMV_FORMATS for n, K, N in GPT2_SHAPES]
        cases.append(("int8-ch head", 768, 50257, 8, 0))
        cases.insert(0, ("warm-up", 768, 2304, 4, 32))  # first launches of the process, not reported

        def timed(fn, n):
            return graph_us(torch, ctx, stream, fn, max(n, 64))

        for name, K, N, bits, group in cases:
            src = torch.randn((K, N), device="cuda", generator=g) * 0.02
            w = lm.HipQuantMatrix.from_f32(ctx, src, bits, group, False, True)
            nb = w.nbytes()
            nrot = max(2, -(-rot_bytes // nb))
            x = torch.randn((1, K), device="cuda", generator=g)
            out = torch.empty((1, N), device="cuda")
            alg = nb + 2 * K + 4 * N
            torch.cuda.nvtx.range_push(f"c1 {name} llc")  # (a marker range for kernel traces)
            us = timed(lambda i: lm.linear(ctx, out, x, w), 1)
            torch.cuda.nvtx.range_pop()
            if name == "warm-up":
                w.free()
                continue
            ws = [w] + [lm.HipQuantMatrix.from_f32(ctx, src, bits, group, False, True) for _ in range(nrot - 1)]
            torch.cuda.nvtx.range_push(f"c1 {name} hbm")
            us_hbm = timed(lambda i: lm.linear(ctx, out, x, ws[i % nrot]), nrot)
            torch.cuda.nvtx.range_pop()
            for m in ws:
                m.free()
            llc_floor = min(read_floor(torch, lm, ctx, stream, nb, 1, grid=gr, reps=64, graph=True)
                            for gr in (256, 1024, 2048))
            hbm_floor = min(read_floor(torch, lm, ctx, stream, nb, nrot, grid=gr, reps=nrot, graph=True)
                            for gr in (256, 1024, 2048))
            res[name] = {"llc_us": round(us, 2), "llc_gbs": round(alg / us / 1e3, 1),
                         "llc_floor_us": round(llc_floor, 2),
                         "hbm_us": round(us_hbm, 2), "hbm_gbs": round(alg / us_hbm / 1e3, 1),
                         "hbm_floor_us": round(hbm_floor, 2)}
    ctx.set_stream(None)
    return res


PREFILL_T = 476
F16_MFMA_PEAK = 2.5e15   # dense fp16 MFMA flop/s of MI355X
LAYER_SHAPES = [("qkv", 768, 2304), ("proj", 768, 768), ("fc", 768, 3072), ("fcproj", 3072, 768)]


def prefill(torch, lm, synth, ctx, tensors, model4, reps=5):
    """Config 3: a 476-token prompt through the GPT-2 weights in int4-g32 and
    int8-g32 A16 form (tok/s = T / prefill span, gpt2t.mojo:949-967), and the
    four layer GEMMs alone at M = 476: time, algorithmic int16 x intN ops
    (2 M K N) and executed matrix-core ops against their peak: both forms
    on the fp16 matrix cores (the hi / lo activation planes: 2 products per
    MAC, M padded to 16, against 2.5 PFLOP/s)."""
    prompt = synth.prompt_ids(1337, PREFILL_T)
    res = {}
    for bits in (4, 8):
        m = model4 if bits == 4 else lm.GPT2(ctx, tensors, bits=8, group=32)
        ms = []
        for _ in range(reps + 1):
            _, p_ms, _ = m.generate(prompt, 1)
            ms.append(p_ms)
        if bits == 8:
            m.free()
        ms = sorted(ms[1:])
        res[f"int{bits}_g32_tok_s"] = round(PREFILL_T / (ms[len(ms) // 2] / 1000.0), 1)
        res[f"int{bits}_g32_ms"] = round(ms[len(ms) // 2], 3)
    stream = torch.cuda.Stream()
    gemm = {}
    with torch.cuda.stream(stream):
        ctx.set_stream(stream)
        g = torch.Generator(device="cuda").manual_seed(3003)
        for bits in (4, 8):
            tot_us, alg, exe = 0.0, 0, 0
            for name, K, N in LAYER_SHAPES:
                w = lm.HipQuantMatrix.from_f32(ctx, torch.randn((K, N), device="cuda", generator=g) * 0.02, bits, 32,
                                               False, True)
                x = torch.randn((PREFILL_T, K), device="cuda", generator=g)
                out = torch.empty((PREFILL_T, N), device="cuda")
                for _ in range(3):
                    lm.linear(ctx, out, x, w)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for _ in range(20):
                    lm.linear(ctx, out, x, w)
                e1.record(stream)
                e1.synchronize()
                us = e0.elapsed_time(e1) * 1000.0 / 20
                w.free()
                tot_us += us
                alg += 2 * PREFILL_T * K * N
                exe += 2 * (-(-PREFILL_T // 16) * 16) * N * K * 2
                gemm[f"int{bits}_{name}_us"] = round(us, 2)
            gemm[f"int{bits}_layer_us"] = round(tot_us, 2)
            gemm[f"int{bits}_alg_tops"] = round(alg / tot_us / 1e6, 1)
            gemm[f"int{bits}_mfma_util"] = round(exe / (tot_us * 1e-6) / F16_MFMA_PEAK, 4)
    ctx.set_stream(None)
    res["layer_gemms_m476"] = gemm
    return res


def int_attention(lm, synth, ctx, tensors, model, steps):
    """--attention int (IntAttnKV, gpt2t.mojo:1251-1257): decode tok/s of
    config 0's generation with integer attention beside float attention, after
    the 12-token prompt and after a 476-token one (where attention reads
    ~500 cached positions per layer and head)."""
    mi = lm.GPT2(ctx, tensors, attention="int")
    res = {}
    for name, plen in (("prompt12", PROMPT), ("prompt476", PREFILL_T)):
        prompt = synth.prompt_ids(SEED, plen)
        for tag, m in (("float", model), ("int", mi)):
            m.generate(prompt, GEN)  # warm-up (captures the decode graph)
            n, dms = 0, 0.0
            for _ in range(steps):
                toks, _, d = m.generate(prompt, GEN)
                n += len(toks)
                dms += d
            res[f"{tag}_{name}_decode_tok_s"] = round(n / (dms / 1000.0), 1)
    mi.free()
    return res


# README.md:75-90's QuantMatrix rows: --dtype, --head int8, the reference's
# decode tok/s short / long on its CPU
FORMAT_ROWS = [("int8-ch", (200, 175)), ("int4-g32", (150, 136)), ("int8-ch-a16", (283, 241)),
               ("int4-ch-a16", (251, 214))]


def format_table(lm, synth, ctx, tensors, steps):
    """Decode tok/s of config 0's generation for the other QuantMatrix
    formats of the reference's table (float activations and A16), after the
    12-token prompt and after a 476-token one."""
    res = {}
    for dtype, ref in FORMAT_ROWS:
        m = lm.GPT2(ctx, tensors, dtype=dtype, head="int8")
        row = {"reference_cpu": ref}
        for name, plen in (("prompt12", PROMPT), ("prompt476", PREFILL_T)):
            prompt = synth.prompt_ids(SEED, plen)
            m.generate(prompt, GEN)  # warm-up (captures the decode graph)
            n, dms = 0, 0.0
            for _ in range(steps):
                toks, _, d = m.generate(prompt, GEN)
                n += len(toks)
                dms += d
            row[f"{name}_decode_tok_s"] = round(n / (dms / 1000.0), 1)
        res[dtype] = row
        m.free()
    return res


GGUF_KINDS = {"Q4_0": 2, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "Q8_0": 8}
GGUF_SHAPES = [(4096, 4096), (4096, 11008), (11008, 4096), (4096, 32000)]


def gguf_sweep(torch, lm, synth, ctx, rot_bytes=512 << 20):
    """Config 2: the GGUF decode GEMV (float activations, batch 1) at the
    Llama shapes K x N, over distinct weight buffers totalling > 512 MiB (twice
    the Infinity Cache); GB/s of nbytes + 4K + 4N per launch."""
    res = {}
    stream = torch.cuda.Stream()
    for name, t in GGUF_KINDS.items():
        for K, N in GGUF_SHAPES:
            bs, bb = synth.GGUF_BLOCK[t]
            nbytes = N * (K // bs) * bb
            nbuf = max(2, min(48, -(-rot_bytes // nbytes)))
            base = synth.gguf_blocks(t, N, K, seed=7)
            mats = [lm.HipGGUFMatrix.from_blocks(ctx, t, base, N, K) for _ in range(nbuf)]
            with torch.cuda.stream(stream):
                ctx.set_stream(stream)
                x = torch.randn((1, K), device="cuda")
                out = torch.empty((1, N), device="cuda")
                for i in range(2 * nbuf):
                    lm.linear(ctx, out, x, mats[i % nbuf])
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                reps = 8 * nbuf
                e0.record(stream)
                for i in range(reps):
                    lm.linear(ctx, out, x, mats[i % nbuf])
                e1.record(stream)
                e1.synchronize()
            ctx.set_stream(None)
            us = e0.elapsed_time(e1) * 1000.0 / reps
            alg = nbytes + 4 * K + 4 * N
            res[f"{name} {K}x{N}"] = {"us": round(us, 2), "gbs": round(alg / us / 1e3, 1),
                                      "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4)}
            log(name, K, N, res[f"{name} {K}x{N}"])
            for m in mats:
                m.free()
    return res


LLAMA_PROMPT, LLAMA_GEN, LLAMA_SEED = 1024, 128, 4004


def llama_kernels(torch, lm, synth, ctx, nbuf=8, reps=40):
    """Config 4's matrix kernels called directly through the C ABI (for
    counter passes): the Q6_K 32000 x 2048 int16 head at 1 and 16 tokens,
    and the Q4_K gate / up matrix (11264 x 2048) at 1, 16 and 1024 tokens
    (one-token GEMV; fp16 matrix-core matmul over its activation record;
    the LDS-staged form for 64+ tokens), each over nbuf rotated copies."""
    cfg = lm.TINYLLAMA
    res = {}
    stream = torch.cuda.Stream()
    for name, t, N, K, Ts in (("head Q6_K", 14, cfg["vocab"], cfg["dim"], (1, 16)),
                              ("gate/up Q4_K", 12, 2 * cfg["ffn"], cfg["dim"], (1, 16, 1024))):
        base = synth.gguf_blocks(t, N, K, seed=5, scale=2e-5 if t == 14 else 1e-4)
        mats = [lm.HipGGUFMatrix.from_blocks(ctx, t, base, N, K) for _ in range(nbuf)]
        with torch.cuda.stream(stream):
            ctx.set_stream(stream)
            for T in Ts:
                x = torch.randn((T, K), device="cuda")
                out = torch.empty((T, N), device="cuda")
                fn = (lambda i: lm.head(ctx, out, x, mats[i % nbuf])) if t == 14 else \
                     (lambda i: lm.linear(ctx, out, x, mats[i % nbuf]))
                for i in range(nbuf):
                    fn(i)
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(reps):
                    fn(i)
                e1.record(stream)
                e1.synchronize()
                res[f"{name} T={T}"] = round(e0.elapsed_time(e1) * 1000.0 / reps, 2)
        ctx.set_stream(None)
        for m in mats:
            m.free()
    return res


def llama_decode(lm, synth, ctx):
    """Config 4: the TinyLlama-shaped decoder (Q4_K layers, Q6_K head, int8
    KV cache) with seeded random weights; a 1024-token random prompt per
    sequence, then 128 greedy tokens at batch 1 and batch 16.  tok/s as the
    reference defines it: generated tokens after the first (the decode steps)
    over the decode span, summed over the batch."""
    cfg = dict(lm.TINYLLAMA, batch=16)
    m = lm.Llama(ctx, cfg, synth.llama_tensors(cfg, LLAMA_SEED))
    res = {"weight_bytes": int(m.weight_bytes())}
    # bytes one decode step reads at batch 1: every matrix but the embedding
    # (one row), and the cache up to the mean position
    embd = cfg["vocab"] * (cfg["dim"] // 256) * 144
    kv_pos = cfg["n_layer"] * cfg["n_kv"] * 2 * (64 + 4)
    mean_pos = LLAMA_PROMPT + (LLAMA_GEN - 1) / 2
    step_bytes = res["weight_bytes"] - embd + embd // cfg["vocab"] + kv_pos * mean_pos
    for B in (1, 16):
        prompts = synth.llama_prompts(LLAMA_SEED, B, LLAMA_PROMPT, cfg["vocab"])
        m.generate(prompts, 8)  # warm: graph capture
        toks, pre_ms, dec_ms = m.generate(prompts, LLAMA_GEN)
        tok_s = B * (LLAMA_GEN - 1) / (dec_ms / 1000.0)
        res[f"bs{B}_decode_tok_s"] = round(tok_s, 1)
        res[f"bs{B}_ms_per_step"] = round(dec_ms / (LLAMA_GEN - 1), 3)
        res[f"bs{B}_prefill_tok_s"] = round(B * LLAMA_PROMPT / (pre_ms / 1000.0), 1)
        if B == 1:
            res["bs1_decode_gbs_effective"] = round(step_bytes * tok_s / 1e9, 1)
    m.free()
    return res


def host_cpu():
    """lscpu's model name and topology, and the CPU share this process may use."""
    info = {"model": None, "sockets": None, "cores_per_socket": None, "threads_per_core": None}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            v = v.strip()
            if k == "Model name":
                info["model"] = v
            elif k == "Socket(s)" and v.isdigit():
                info["sockets"] = int(v)
            elif k == "Core(s) per socket" and v.isdigit():
                info["cores_per_socket"] = int(v)
            elif k == "Thread(s) per core" and v.isdigit():
                info["threads_per_core"] = int(v)
    except (OSError, subprocess.SubprocessError):
        pass
    allowed = len(os.sched_getaffinity(0))
    tpc = info["threads_per_core"] or 1
    info["physical_cores"] = (info["sockets"] or 1) * (info["cores_per_socket"] or allowed)
    info["smt"] = tpc > 1
    info["cpus_allowed"] = allowed
    # one thread per physical core of what this process may use, within the
    # box's CPU share for one GPU (16)
    info["share"] = max(1, min(16, allowed // tpc if tpc > 1 else allowed, info["physical_cores"]))
    return info


def cpu_baseline(tensors, prompt):
    """The CPU baseline: the reference's team decode (gpt2t.mojo:350-447)
    restated in C with VPDPWSSD dots (oracle/llmq_oracle.c orc_cpu_*,
    bit-identical to the scalar oracle), on this host: greedy decode of GEN
    tokens after the prompt, tok/s as the reference defines it (generated
    tokens / the decode loop's wall time), for a sweep of team sizes; the
    headline is one thread per physical core (the reference's default,
    gpt2t.mojo:277-281) within the box's CPU share."""
    import oracle
    from llm_mojo_amd import gpt2

    host = host_cpu()
    nt = host["share"]
    oracle.set_threads(nt)
    m = oracle.GPT2(gpt2.params_list(tensors))
    vnni = bool(oracle.cpu_vnni())
    sweep, prompt_s = {}, None
    for t in sorted({1, 4, 8, 16, nt}):
        if t > nt:
            continue
        toks, ps, ds = m.cpu_generate(prompt, GEN, t)
        sweep[t] = round(len(toks) / ds, 1)
        prompt_s = ps
        log(f"cpu baseline: {t} threads {sweep[t]} tok/s")
    best = max(sweep, key=sweep.get)
    head_ms = round(m.cpu_head_seconds(min(4, nt), 30) * 1e3, 3)
    extra = cpu_kernels(oracle, tensors, nt)
    return {"value": sweep[nt], "unit": "tok/s", "cores": nt, "kind": "port",
            "label": "C restatement of llm_mojo's CPU path",
            "sample": f"GPT-2 124M int4-g32-a16 (int8-ch head, int8 KV): {len(prompt)}-token prompt through the "
                      f"oracle's forward ({prompt_s * 1e3:.0f} ms, scalar), then {GEN} greedy tokens through the team "
                      f"decode with {'VPDPWSSD (AVX-512 VNNI)' if vnni else 'the portable scalar path (no AVX-512 VNNI)'}"
                      f" on {nt} threads",
            "vnni": vnni, "threads_sweep_tok_s": sweep, "best": {"threads": best, "tok_s": sweep[best]},
            "head_int8_ch_ms": {"threads": min(4, nt), "ms": head_ms, "reference_4t_ms": "0.96-1.00"},
            **extra, "host": host}


def cpu_kernels(oracle, tensors, nt, reps=100, rot_bytes=256 << 20):
    """The CPU baseline's per-config kernels on nt threads, beside the GPU's:
    config 3's 476-token prompt (Model.forward with tile_i16 on VPDPWSSD,
    kernels.mojo:512-573, and the vector attention; median of 3 after a
    warm-up), config 1's one-token GEMVs (linear_team, kernels.mojo:774-866,
    with dot_row_i16's VNNI branches) and config 2's GGUF GEMVs (dot_row's
    block decoders on AVX-512, gguf.mojo:178-297, 388-417): median of `reps`
    calls over copies totalling >= rot_bytes, so codes come from memory.
    Every form is bit-identical to the scalar oracle (tests/)."""
    import numpy as np

    from llm_mojo_amd import gpt2, synth

    res = {}
    m = oracle.GPT2(gpt2.params_list(tensors))
    prompt = synth.prompt_ids(SEED, PREFILL_T)
    secs = []
    for _ in range(4):
        _, s = m.cpu_prompt(prompt, nt)
        secs.append(s)
    s = sorted(secs[1:])[1]
    res["prompt_476"] = {"tok_s": round(PREFILL_T / s, 1), "ms": round(s * 1e3, 1), "threads": nt}
    log("cpu baseline: 476-token prompt", res["prompt_476"])
    rng = np.random.default_rng(1001)
    g1 = {}
    cases = [(f"int{b}-g{gr} {n}", K, N, b, gr) for b, gr in GEMV_FORMATS for n, K, N in GPT2_SHAPES]
    cases.append(("int8-ch head", 768, 50257, 8, 0))
    for name, K, N, bits, group in cases:
        w = rng.normal(0, 0.02, (K, N)).astype(np.float32)
        q = oracle.QuantMatrix.from_f32(w, bits, group, False, True)
        mats = [q] + [q.clone() for _ in range(max(1, rot_bytes // max(1, q.nbytes())) - 1)]
        x = rng.normal(0, 1, (1, K)).astype(np.float32)
        sec, _ = oracle.cpu_gemv_seconds(mats, x, nt, reps)
        g1[name] = round(sec * 1e3, 4)
        del mats
    res["gemv_cfg1_ms"] = g1
    log("cpu baseline: config-1 GEMVs (ms)", g1)
    g2 = {}
    for tname, t in GGUF_KINDS.items():
        for K, N in GGUF_SHAPES:
            bs, bb = synth.GGUF_BLOCK[t]
            base = synth.gguf_blocks(t, N, K, seed=7)
            copies = [base] + [base.copy() for _ in range(max(1, rot_bytes // base.nbytes) - 1)]
            x = rng.normal(0, 1, K).astype(np.float32)
            sec, _ = oracle.cpu_gguf_gemv_seconds(t, copies, N, K, x, nt, reps)
            g2[f"{tname} {K}x{N}"] = round(sec * 1e3, 3)
            del copies
    res["gguf_cfg2_ms"] = g2
    log("cpu baseline: config-2 GGUF GEMVs (ms)", g2)
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 476-token prefill (config 3)")
    ap.add_argument("--no-llama", action="store_true", help="skip the TinyLlama-shaped decoder (config 4)")
    ap.add_argument("--no-gguf-sweep", action="store_true", help="skip the GGUF GEMV sweep (config 2)")
    ap.add_argument("--no-intattn", action="store_true", help="skip the integer-attention decode comparison")
    ap.add_argument("--no-formats", action="store_true", help="skip the decode table of the other formats")
    ap.add_argument("--no-read-sweep", action="store_true", help="skip the pure-read size sweep")
    ap.add_argument("--micro-only", action="store_true",
                    help="only config 1's GEMVs and the read sweep (for rocprofv3 runs)")
    ap.add_argument("--gguf-only", action="store_true",
                    help="only config 2's GGUF GEMV sweep and the 1 GiB reference copy (for rocprofv3 runs)")
    ap.add_argument("--llama-only", action="store_true",
                    help="only config 4's decoder and the 1 GiB reference copy (for rocprofv3 runs)")
    ap.add_argument("--prefill-only", action="store_true",
                    help="only config 3's 476-token prompts and layer GEMMs (for rocprofv3 runs)")
    ap.add_argument("--llama-kernels", action="store_true",
                    help="only config 4's head and gate/up kernels through the C ABI, and the 1 GiB reference copy")
    ap.add_argument("--roofline-only", action="store_true",
                    help="only the roofline GEMV and the reference copy (for rocprofv3 --pmc runs)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import llm_mojo_amd as lm
    from llm_mojo_amd import synth

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    if args.roofline_only:
        ctx = lm.Context(0)
        r = gemv_roofline(torch, lm, ctx)
        print(json.dumps({"roofline_kernel": r, "copy_gbs": round(copy_bandwidth(torch), 1)}), flush=True)
        return
    if args.gguf_only or args.llama_only or args.llama_kernels:
        ctx = lm.Context(0)
        out = {"copy_gbs": round(copy_bandwidth(torch), 1)}
        if args.llama_kernels:
            out["llama_kernels_us"] = llama_kernels(torch, lm, synth, ctx)
        if args.gguf_only:
            out["gguf_gemv_sweep"] = gguf_sweep(torch, lm, synth, ctx)
        if args.llama_only:
            out["tinyllama_q4k_q6k"] = llama_decode(lm, synth, ctx)
        print(json.dumps(out), flush=True)
        return
    if args.micro_only:
        ctx = lm.Context(0)
        out = {"gemv_micro_llc": gemv_micro(torch, lm, ctx)}
        if not args.no_read_sweep:
            out["read_sweep"] = read_sweep(torch, lm, ctx)
        print(json.dumps(out), flush=True)
        return
    log("generating synthetic GPT-2 weights")
    tensors = synth.gpt2_tensors(SEED)
    prompt = synth.prompt_ids(SEED, PROMPT)
    ctx = lm.Context(0)
    model = lm.GPT2(ctx, tensors)
    if args.prefill_only:
        print(json.dumps({"prefill_476": prefill(torch, lm, synth, ctx, tensors, model)}), flush=True)
        return
    log("model", model.name(), "weight bytes", model.weight_bytes())

    for _ in range(args.warmup):
        model.generate(prompt, GEN)
    torch.cuda.synchronize()
    gen_total, dec_ms, pre_ms = 0, 0.0, 0.0
    t0 = time.perf_counter()
    for _ in range(args.steps):
        toks, p_ms, d_ms = model.generate(prompt, GEN)
        gen_total += len(toks)
        dec_ms += d_ms
        pre_ms += p_ms
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    tok_s = gen_total / (dec_ms / 1000.0)
    log(f"decode {tok_s:.0f} tok/s, prefill {PROMPT * args.steps / (pre_ms / 1000.0):.0f} tok/s, "
        f"wall {wall * 1000 / args.steps:.2f} ms/step")

    roof = None
    extra = {}
    if not args.no_roofline:
        r = gemv_roofline(torch, lm, ctx)
        traffic, trace_us = measured_traffic()
        roof = {"bound": "hbm", "achieved": round(r["gbs"], 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(r["gbs"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                "timing": "HIP events over 3 replays of a HIP graph of 144 launches on the kernel's stream (36 "
                          "rotated weight buffers, 965 MB); a launch's dispatch overlaps the previous one's tail, so "
                          "this sits below a single dispatch's start-to-end time in a kernel trace (trace_avg_us)"}
        if trace_us:
            roof["trace_avg_us"] = trace_us
            roof["trace_frac"] = round(r["alg_bytes"] / trace_us / 1e3 / HBM_PEAK_GBS, 4)
        r["traffic_source"] = ("profiles/gemv_a16_int4_g32_4096x11008.traffic.json: rocprofv3 --pmc FETCH_SIZE "
                               "and WRITE_SIZE of this kernel, scaled by the same counters on a copy of known size")
        extra["roofline_kernel"] = r
        extra["copy_gbs"] = round(copy_bandwidth(torch), 1)
        log("gemv", r, "copy GB/s", extra["copy_gbs"])
    # bytes a decode token reads (weights + KV at the mean position)
    mean_pos = PROMPT + (GEN - 1) / 2
    token_bytes = model.weight_bytes() - 4 * 1024 * 768 + 3072 + 19584 * (mean_pos + 1) + 19584
    extra["decode_bytes_per_token"] = int(token_bytes)
    extra["decode_gbs_effective"] = round(token_bytes * tok_s / 1e9, 1)

    if not args.no_read_sweep:
        log("read sweep")
        extra["read_sweep"] = read_sweep(torch, lm, ctx)
    log("gemv micro")
    extra["gemv_micro_llc"] = gemv_micro(torch, lm, ctx)
    if not args.no_intattn:
        log("integer attention decode")
        extra["gpt2_int_attention"] = int_attention(lm, synth, ctx, tensors, model, args.steps)
        log(extra["gpt2_int_attention"])
    if not args.no_formats:
        log("format table")
        extra["gpt2_formats"] = format_table(lm, synth, ctx, tensors, args.steps)
        log(extra["gpt2_formats"])
    if not args.no_prefill:
        log("prefill 476")
        extra["prefill_476"] = prefill(torch, lm, synth, ctx, tensors, model)
        log(extra["prefill_476"])
    if not args.no_llama:
        log("tinyllama-shaped decode")
        extra["tinyllama_q4k_q6k"] = llama_decode(lm, synth, ctx)
        log(extra["tinyllama_q4k_q6k"])
    if not args.no_gguf_sweep:
        log("gguf sweep")
        extra["gguf_gemv_sweep"] = gguf_sweep(torch, lm, synth, ctx)

    cpu = None
    if not args.no_cpu:
        try:
            log("cpu baseline")
            cpu = cpu_baseline(tensors, prompt)
            cpu["value"] = round(cpu["value"], 2)
        except Exception as e:  # the baseline is reported, not required
            log("cpu baseline failed:", repr(e))

    line = {
        "metric": "decode tok/s (GPT-2 int4-g32-a16, bs1) + W4A16 GEMV achieved GB/s vs HBM peak",
        "value": round(tok_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall * 1000 / args.steps, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int16xint4->int32",
        "data": "synthetic (seeded random-init GPT-2 124M weights, random prompt ids)",
        "config": {"workload": "GPT-2 124M int4-g32-a16 + int8-ch head + int8 KV, bs1, 12-token prompt "
                               "then 100 greedy tokens (BASELINE config 0)",
                   "global_batch": 1, "prompt": PROMPT, "generated": GEN, "parallelism": "single GPU"},
        "prefill_tok_s": round(PROMPT * args.steps / (pre_ms / 1000.0), 1),
        "roofline": roof,
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
