"""Benchmark of the quantized-linear hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode-w8]

Default workload (`decode-w8`): INT8 per-channel, fp16-activation decode GEMVs over
every linear shape of one 2B-class hybrid layer -- q/o (2048,2048), k/v (2048,512),
gate/up (2048,6144), down (6144,2048), linear-attention in/out (2048,4096) and
(4096,2048) -- plus the vocabulary head (2048,248320), at M = 1, 2 and 4 rows.
One step runs all of them once per M.  The layer weights exist in `--layers`
distinct copies (default 8, about 0.5 GB, like consecutive layers of a model), so
every launch streams its weights from HBM rather than the 256 MB last-level cache.

The layer launches of one M are replayed as one HIP graph; the vocabulary-head
launch stays eager with HIP events around it on its launch stream, which gives the
dominant kernel's live per-launch time for the roofline object.

Other workloads (`--workload`): decode-w4 (same shapes, W4 group 128), prefill
(M in 128/512/2048, TFLOP/s), prefill-9b (the same over 9B-class layer shapes, where
M = 2048 takes the balanced schedule), chain-w4 (9B-class 32-layer W4 decode chain), single
(one 2048x6144 int8 linear, M=1), engine-w8 / engine-w4 (the engine-signature calls
of one layer at decode rows and a 512-row prefill chunk), layout (the load-time layout
producers: GPU requantization and GPTQ / AWQ repacks, HBM GB/s).

Prints ONE JSON line (rank 0).  Synthetic data; weights are random in the engine
layouts.
"""
from __future__ import annotations

import argparse
import importlib.util
import json
import os
import pathlib
import sys
import time

ROOT = pathlib.Path(__file__).resolve().parent
PKG_DIR = ROOT / "qwen_3.5_comfy_prompt_enhancer_amd"
ALIAS = "qwen35_amd"

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 MFMA, TFLOP/s

METRIC = "W8/W4 decode GEMV HBM GB/s (% peak) at M=1-4; prefill GEMM TFLOPS"

LAYER_SHAPES = [  # (name, K, N) of one 2B-class hybrid layer
    ("q", 2048, 2048), ("k", 2048, 512), ("v", 2048, 512), ("o", 2048, 2048),
    ("gate", 2048, 6144), ("up", 2048, 6144), ("down", 6144, 2048),
    ("lin_in", 2048, 4096), ("lin_out", 4096, 2048),
]
HEAD = ("lm_head", 2048, 248320)
CHAIN_SHAPES = [  # 9B-class layer
    ("q", 4096, 4096), ("k", 4096, 1024), ("v", 4096, 1024), ("o", 4096, 4096),
    ("gate", 4096, 12288), ("up", 4096, 12288), ("down", 12288, 4096),
]
CHAIN_HEAD = ("lm_head", 4096, 248320)
# Dependency level of each linear within a decode layer, as a real decode step orders
# them: the projections that read the layer input, then the ones that read the
# attention / linear-attention output, then gate/up (after the residual and norm),
# then down; the next layer reads down's result, the vocabulary head the last layer's.
LAYER_LEVEL = {"q": 0, "k": 0, "v": 0, "lin_in": 0, "o": 1, "lin_out": 1, "gate": 2, "up": 2, "down": 3}
LEVELS_PER_LAYER = 4
PREFILL_SHAPES = [("gate", 2048, 6144), ("down", 6144, 2048), ("q", 2048, 2048)]
# 9B-class layer (hidden 4096, intermediate 12288): at M = 2048 the gate shape has 384
# tiles of 256x256, one and a half rounds of the chip, and takes the balanced schedule
PREFILL_SHAPES_9B = [("gate", 4096, 12288), ("down", 12288, 4096), ("q", 4096, 4096)]


def _load_package():
    if ALIAS in sys.modules:
        return sys.modules[ALIAS]
    spec = importlib.util.spec_from_file_location(
        ALIAS, PKG_DIR / "__init__.py", submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[ALIAS] = mod
    spec.loader.exec_module(mod)
    return mod


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ algorithmic bytes

def bytes_w8(M, K, N):
    """int8 weights + fp16 per-column scales + fp16 activations in + fp16 out."""
    return K * N + 2 * N + 2 * M * K + 2 * M * N


def bytes_w4(M, K, N, G=128):
    """packed nibbles + fp16 group scales + fp16 activations in + fp16 out."""
    return K * N // 2 + 2 * (K // G) * N + 2 * M * K + 2 * M * N


def _capture(g):
    """HIP graph capture on a stream that has a split-K workspace (kernels/qlin.py)."""
    from qwen35_amd.kernels import qlin
    return qlin.capture(g)


# ------------------------------------------------------------------ weights

class Weights:
    def __init__(self, kind, K, N, dev, gen, group=128):
        import torch
        self.kind, self.K, self.N = kind, K, N
        if kind == "w8":
            self.w = torch.randint(-127, 128, (K, N), generator=gen, dtype=torch.int8).to(dev)
            self.s = ((torch.randn(N, generator=gen) * 0.02).abs() / 127).to(torch.float16).to(dev)
        else:
            self.w = torch.randint(0, 256, (K // 2, N), generator=gen, dtype=torch.uint8).to(dev)
            self.s = ((torch.randn((K // group, N), generator=gen) * 0.02).abs() / 7).to(torch.float16).to(dev)

    def run(self, lin, x, out):
        if self.kind == "w8":
            lin.linear_w8(x, self.w, self.s, out)
        else:
            lin.linear_w4(x, self.w, self.s, out)

    def nbytes(self, M):
        return bytes_w8(M, self.K, self.N) if self.kind == "w8" else bytes_w4(M, self.K, self.N)


# ------------------------------------------------------------------ decode sweep

def decode_sweep(args, kind, shapes, head, ms, layers, reuse=None):
    """Returns (total_bytes_per_step, step_fn, head_events, head_bytes_by_m, record, ctx);
    `reuse` = the ctx of an earlier call with the same shapes (its weights and buffers)."""
    import torch
    dev = torch.device("cuda", 0)
    lin = importlib.import_module(f"{ALIAS}.kernels.linear")
    if reuse is not None:
        lw, hw, xs, outs, hout = reuse[:5]
    else:
        gen = torch.Generator().manual_seed(1234)
        lw = [[Weights(kind, K, N, dev, gen) for (_, K, N) in shapes] for _ in range(layers)]
        hw = Weights(kind, head[1], head[2], dev, gen)
        kmax = max([K for _, K, _ in shapes] + [head[1]])
        xs = {M: torch.randn((M, kmax), generator=gen).to(torch.float16).to(dev) for M in ms}
        # every job writes an output of its own (layer copy l, shape i), so a launch of
        # the whole sweep is a valid computation whose results are checked below
        outs = {M: [[torch.empty((M, N), dtype=torch.float16, device=dev) for (_, _, N) in shapes]
                    for _ in range(layers)] for M in ms}
        hout = {M: torch.empty((M, head[2]), dtype=torch.float16, device=dev) for M in ms}

    def xin(M, K):
        return xs[M][:, :K]

    def run_layers(M):
        for l in range(layers):
            for i, (_, K, _) in enumerate(shapes):
                lw[l][i].run(lin, xin(M, K), outs[M][l][i])

    total = sum((layers * sum(w.nbytes(M) for w in lw[0]) if lw else 0) + hw.nbytes(M) for M in ms)
    if args.launch == "chain":
        # one persistent launch per M: every layer copy and the head, in dependency
        # levels (args.levels == "layer") or all independent ("flat")
        from qwen35_amd.kernels.chain import DecodeChain
        order = sorted(range(len(shapes)), key=lambda i: LAYER_LEVEL.get(shapes[i][0], 0))
        chains = {}
        for M in ms:
            ch = DecodeChain(M)
            base = 0
            for l in range(layers):
                for i in order:
                    _, K, _ = shapes[i]
                    lvl = base + LAYER_LEVEL.get(shapes[i][0], 0) if args.levels == "layer" else 0
                    ch.add(xin(M, K), lw[l][i].w, lw[l][i].s, outs[M][l][i], level=lvl)
                if shapes and args.levels == "layer":
                    base += LEVELS_PER_LAYER
            if args.head == "chain":
                ch.add(xin(M, head[1]), hw.w, hw.s, hout[M],
                       level=(base if shapes and args.levels == "layer" else 0))
            ch.build()
            chains[M] = ch
        for M in ms:
            chains[M].run()
        torch.cuda.synchronize()
        ev = {M: [] for M in ms}
        record = {"on": False}

        # with --head own the vocabulary head follows the chain as its own launch on the
        # same stream (the wide GEMV plan; the stream order is its dependency)
        head_own = args.head == "own"
        head_graphs = {}
        if head_own:
            # warm-up (allocates the workspace outside capture), then one HIP graph per M:
            # replaying it costs the host one call, so the GPU does not wait for the host
            # between the chain and the head
            for M in ms:
                hw.run(lin, xin(M, head[1]), hout[M])
            torch.cuda.synchronize()
            for M in ms:
                gh = torch.cuda.CUDAGraph()
                with _capture(gh):
                    hw.run(lin, xin(M, head[1]), hout[M])
                head_graphs[M] = gh
            torch.cuda.synchronize()

        # each chain's launch bound once (library function, plan pointer, stream), so
        # the event interval around a launch holds no Python work beyond the call
        from qwen35_amd.kernels import qlin as C
        launch = {M: (C.lib().qlin_chain_run, chains[M].plan.data_ptr(), torch.cuda.current_stream().cuda_stream)
                  for M in ms}

        def run_chain(M):
            fn, plan, stream = launch[M]
            rc = fn(plan, stream)
            if rc != 0:
                C.check(rc, "qlin_chain_run")

        def step():
            for M in ms:
                if record["on"]:
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record()
                    run_chain(M)
                    e1.record()
                    ev[M].append((e0, e1))
                else:
                    run_chain(M)
                if head_own:
                    head_graphs[M].replay()

        step_bytes = {M: (layers * sum(w.nbytes(M) for w in lw[0]) if lw else 0)
                      + (0 if head_own else hw.nbytes(M)) for M in ms}
        return total, step, ev, step_bytes, record, (lw, hw, xs, outs, hout, lin, chains)

    # eager warm-up (allocates the workspace outside capture), then capture per M
    for M in ms:
        run_layers(M)
        hw.run(lin, xin(M, head[1]), hout[M])
    torch.cuda.synchronize()
    graphs = {}
    if not args.no_graph:
        for M in ms:
            g = torch.cuda.CUDAGraph()
            with _capture(g):
                run_layers(M)
            graphs[M] = g
        torch.cuda.synchronize()

    head_ev = {M: [] for M in ms}
    record = {"on": False}

    def step():
        for M in ms:
            if graphs:
                graphs[M].replay()
            else:
                run_layers(M)
            if record["on"]:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record()
                hw.run(lin, xin(M, head[1]), hout[M])
                e1.record()
                head_ev[M].append((e0, e1))
            else:
                hw.run(lin, xin(M, head[1]), hout[M])

    head_bytes = {M: hw.nbytes(M) for M in ms}
    return total, step, head_ev, head_bytes, record, (lw, hw, xs, outs, hout, lin, None)


def time_steps(step, steps, warmup, record=None, span=None):
    """Seconds per step over `steps` timed steps after `warmup` untimed ones.  With
    `record`, the step records its per-launch events while timed; with `span` (a dict),
    one HIP event pair on the current stream brackets the timed steps and span["ms"]
    receives its elapsed time (no event inside the region)."""
    import torch
    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    if record is not None:
        record["on"] = True
    if span is not None:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    if span is not None:
        e0.record()
    for _ in range(steps):
        step()
    if span is not None:
        e1.record()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    if record is not None:
        record["on"] = False
    if span is not None:
        span["ms"] = e0.elapsed_time(e1)
    return (t1 - t0) / steps


def detail_table(ctx, kind, shapes, head, ms, reps=40):
    """Per-shape GPU time (stderr only): a HIP graph of `reps` launches of one shape,
    rotating over the layer copies, timed with events around its replay."""
    import torch
    lw, hw, xs, outs, hout, lin, _ = ctx
    layers = max(1, len(lw))
    rows = []
    for M in ms:
        for i, (name, K, N) in enumerate(list(shapes) + [head]):
            is_head = i == len(shapes)
            n = 4 if is_head else reps

            def body():
                for r in range(n):
                    w = hw if is_head else lw[r % layers][i]
                    w.run(lin, xs[M][:, :K], hout[M] if is_head else outs[M][r % layers][i])
            body()
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with _capture(g):
                body()
            g.replay()
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(3):
                g.replay()
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / (3 * n)
            b = (hw if is_head else lw[0][i]).nbytes(M)
            rows.append((M, name, K, N, us, b / us / 1e3))
    log(f"{'M':>2} {'shape':>8} {'K':>6} {'N':>7} {'us':>9} {'GB/s':>8} {'%peak':>6}")
    for M, name, K, N, us, gbs in rows:
        log(f"{M:>2} {name:>8} {K:>6} {N:>7} {us:9.2f} {gbs:8.0f} {100 * gbs / HBM_PEAK_GBS:6.1f}")


# ------------------------------------------------------------------ prefill

def prefill_bench(args, shapes=PREFILL_SHAPES):
    import torch
    dev = torch.device("cuda", 0)
    lin = importlib.import_module(f"{ALIAS}.kernels.linear")
    gen = torch.Generator().manual_seed(99)
    ms = [128, 512, 2048]
    # The weights exist in several copy sets (about 45 MB each, > 512 MB in all) and
    # consecutive steps use different sets, so every step streams its weights from
    # HBM rather than the 256 MB last-level cache, as consecutive layers would.
    set_bytes = sum(bytes_w8(0, K, N) + bytes_w4(0, K, N) for (_, K, N) in shapes)
    nsets = max(1, -(-600_000_000 // set_bytes))
    xs = {}
    outs = {}
    for (name, K, N) in shapes:
        for M in ms:
            if (K, M) not in xs:
                xs[(K, M)] = torch.randn((M, K), generator=gen).to(torch.float16).to(dev)
            if (N, M) not in outs:
                outs[(N, M)] = torch.empty((M, N), dtype=torch.float16, device=dev)
    sets = []
    for _ in range(nsets):
        items = []
        for kind in ("w4", "w8"):  # W4 first: graph A below then holds most of the step
            for (name, K, N) in shapes:
                w = Weights(kind, K, N, dev, gen)
                for M in ms:
                    items.append((kind, name, M, K, N, w, xs[(K, M)], outs[(N, M)]))
        sets.append(items)
    items = sets[0]

    # The cases before and after the dominant launch (the largest W8 case: M=2048,
    # 2048x6144) replay as two HIP graphs per copy set; the dominant launch itself runs
    # eagerly between them with HIP events on its launch stream, issued while graph A
    # still occupies the GPU so that no host launch latency enters its timing.
    dom = next(i for i, it in enumerate(items) if it[0] == "w8" and it[2] == 2048 and it[1] == "gate")
    for its in sets:  # eager warm-up (workspace, LDS attributes)
        for (_, _, _, _, _, w, x, o) in its:
            w.run(lin, x, o)
    torch.cuda.synchronize()
    graphs = []
    for its in sets:
        pair = []
        for part in (its[:dom], its[dom + 1:]):
            g = torch.cuda.CUDAGraph()
            with _capture(g):
                for (_, _, _, _, _, w, x, o) in part:
                    w.run(lin, x, o)
            pair.append(g)
        graphs.append(pair)
    torch.cuda.synchronize()
    dom_ev = []
    record = {"on": False}
    state = {"n": 0}

    def step():
        c = state["n"] % nsets
        state["n"] += 1
        dw, dx, do = sets[c][dom][5], sets[c][dom][6], sets[c][dom][7]
        graphs[c][0].replay()
        if record["on"]:
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record()
            dw.run(lin, dx, do)
            e1.record()
            dom_ev.append((e0, e1))
        else:
            dw.run(lin, dx, do)
        graphs[c][1].replay()

    flops = sum(2 * M * K * N for (_, _, M, K, N, _, _, _) in items)
    t = time_steps(step, args.steps, args.warmup, record)
    _, _, M, K, N, _, _, _ = items[dom]
    dur = sum(e0.elapsed_time(e1) for e0, e1 in dom_ev) / len(dom_ev) * 1e-3
    achieved = 2 * M * K * N / dur / 1e12
    roof = {"bound": "mfma", "achieved": round(achieved, 1), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4), "traffic": read_traffic(f"prefill-w8-{M}x{K}x{N}"),
            "kernel": f"prefill_kernel w8 M={M} K={K} N={N}", "flops_per_launch": 2 * M * K * N,
            "avg_launch_us": round(dur * 1e6, 2)}
    if args.detail:
        # per case: one launch per copy set in turn (weights from HBM), HIP events
        for i, (kind, name, M, K, N, _, x, o) in enumerate(items):
            for its in sets:
                its[i][5].run(lin, x, o)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for its in sets:
                its[i][5].run(lin, x, o)
            e1.record()
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) * 1e3 / nsets
            log(f"{kind} {name:>5} M={M:5d} K={K} N={N}: {us:9.1f} us {2 * M * K * N / us / 1e6:8.1f} TFLOP/s")
    return flops, t, roof, nsets


# ------------------------------------------------------------------ engine layer

ENGINE_LAYER = [  # the engine's four quantized calls of one 2B-class layer (engine.py:221-340)
    ("proj3 lin_qkv+lin_z", 2048, 6144 + 2048),
    ("gemm_i8 o + residual", 2048, 2048),
    ("mlp_gate_up_quant", 2048, 2 * 6144),
    ("gemm_i8 down + residual", 6144, 2048),
]


def engine_bench(args, kind, ms=(1, 4, 512)):
    """The engine-signature calls of one layer (int8 activations with per-64 scales,
    bf16 outputs, in-place residuals, the fused gate/up + requantization) over
    `layers` weight copies, at decode rows M = 1, 4 and a prefill chunk M = 512
    (`ms` drops the chunk when only the decode rows are wanted).
    Returns (bytes per step at M = 1, 4; flops per step at M = 512; per-M times)."""
    import torch
    dev = torch.device("cuda", 0)
    gemm = importlib.import_module(f"{ALIAS}.kernels.gemm")
    gen = torch.Generator().manual_seed(77)
    layers = max(1, args.layers)

    def wmat(K, N):
        if kind == "w8":
            return (torch.randint(-127, 128, (K, N), generator=gen, dtype=torch.int8).to(dev),
                    (torch.rand(N, generator=gen) * 1e-3).to(dev), None)
        return (torch.randint(0, 256, (K // 2, N), generator=gen, dtype=torch.uint8).to(dev),
                (torch.rand(K // 128, N, generator=gen) * 1e-3).to(torch.bfloat16).to(dev), None)

    lw = [dict(qkv=wmat(2048, 6144), z=wmat(2048, 2048), o=wmat(2048, 2048), g=wmat(2048, 6144),
               u=wmat(2048, 6144), d=wmat(6144, 2048)) for _ in range(layers)]

    def wbytes(K, N):
        return K * N if kind == "w8" else K * N // 2 + (K // 128) * N * 2

    layer_wbytes = wbytes(2048, 8192) + wbytes(2048, 2048) + 2 * wbytes(2048, 6144) + wbytes(6144, 2048)
    res, pro_res, chain_res = {}, {}, {}
    fused = importlib.import_module(f"{ALIAS}.kernels.fused")
    normk = importlib.import_module(f"{ALIAS}.kernels.norm")
    nw_in = (torch.rand(2048, generator=gen) * 0.1).to(torch.bfloat16).to(dev)
    nw_post = (torch.rand(2048, generator=gen) * 0.1).to(torch.bfloat16).to(dev)

    def timed(run):
        run()
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with _capture(g):
            run()
        for _ in range(args.warmup):
            g.replay()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            g.replay()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / args.steps / layers

    for M in ms:
        a = torch.randint(-127, 128, (M, 2048), generator=gen, dtype=torch.int8).to(dev)
        s = (torch.rand(M, 32, generator=gen) * 1e-2).to(dev)
        a6 = torch.randint(-127, 128, (M, 6144), generator=gen, dtype=torch.int8).to(dev)
        s6 = (torch.rand(M, 96, generator=gen) * 1e-2).to(dev)
        qkvz = torch.empty(M, 8192, dtype=torch.bfloat16, device=dev)
        hid = torch.zeros(M, 2048, dtype=torch.bfloat16, device=dev)
        hq = torch.empty(M, 6144, dtype=torch.int8, device=dev)
        hs = torch.empty(M, 96, dtype=torch.float32, device=dev)
        if kind == "w8":
            fns = (gemm.proj3, gemm.gemm_i8, gemm.mlp_gate_up_quant)
        else:
            w4 = importlib.import_module(f"{ALIAS}.kernels.w4")
            fns = (w4.proj3_w4, w4.gemm_w4, w4.mlp_gate_up_quant_w4)

        def run_layers():
            for L in lw:
                fns[0](a, s, L["qkv"][0], L["qkv"][1], L["z"][0], L["z"][1], None, None, qkvz)
                fns[1](a, s, L["o"][0], L["o"][1], hid, residual=hid)
                fns[2](a, s, L["g"][0], L["g"][1], L["u"][0], L["u"][1], hq, hs)
                fns[1](a6, s6, L["d"][0], L["d"][1], hid, residual=hid)

        res[M] = timed(run_layers)

        # the same layer with its activation producers (engine.py:244-279 with the
        # attention output's gate_mul_quant): producer launches + linears, then the
        # fused calls that make their activations in the linear's own launch
        hid.copy_(torch.randn(M, 2048, generator=gen).to(torch.bfloat16).to(dev))
        aout = (torch.randn(M, 2048, generator=gen)).to(torch.bfloat16).to(dev)
        xq = torch.empty(M, 2048, dtype=torch.int8, device=dev)
        xs = torch.empty(M, 32, dtype=torch.float32, device=dev)

        def run_unfused():
            for L in lw:
                normk.rmsnorm_quant(hid, nw_in, xq, xs, 1e-6)
                fns[0](xq, xs, L["qkv"][0], L["qkv"][1], L["z"][0], L["z"][1], None, None, qkvz)
                normk.gate_mul_quant(aout, qkvz, xq, xs, hd=256)
                fns[1](xq, xs, L["o"][0], L["o"][1], hid, residual=hid)
                normk.rmsnorm_quant(hid, nw_post, xq, xs, 1e-6)
                fns[2](xq, xs, L["g"][0], L["g"][1], L["u"][0], L["u"][1], hq, hs)
                fns[1](hq, hs, L["d"][0], L["d"][1], hid, residual=hid)

        def run_fused():
            for L in lw:
                fused.pro_proj3(fused.Producer.rmsnorm(hid, nw_in, 1e-6), L["qkv"][0], L["qkv"][1], L["z"][0],
                                L["z"][1], None, None, qkvz)
                fused.pro_gemm_i8(fused.Producer.gate_mul(aout, qkvz, hd=256), L["o"][0], L["o"][1], hid,
                                  residual=hid)
                fused.pro_mlp_gate_up_quant(fused.Producer.rmsnorm(hid, nw_post, 1e-6), L["g"][0], L["g"][1],
                                            L["u"][0], L["u"][1], hq, hs)
                fns[1](hq, hs, L["d"][0], L["d"][1], hid, residual=hid)

        pro_res[M] = (timed(run_unfused), timed(run_fused))
        log(f"engine {kind} layer with producers M={M:4d}: {pro_res[M][0] * 1e6:7.1f} us as producer + linear "
            f"launches, {pro_res[M][1] * 1e6:7.1f} us fused")
        if M <= 8:
            # the same layer body as ONE engine-chain launch per layer (kernels/echain.py):
            # o-projection with its gate_mul producer, gate/up + quant with the post-norm,
            # down, the next layer's proj3 with its in-norm (keeping the codes, as the
            # engine's gate_proj reads them); levels 0-3
            echain = importlib.import_module(f"{ALIAS}.kernels.echain")
            chains = []
            for L in lw:
                ch = echain.EngineChain(M)
                ch.gemm_i8(None, None, L["o"][0], L["o"][1], hid, residual=hid,
                           pro=fused.Producer.gate_mul(aout, qkvz, hd=256), level=0)
                ch.mlp_gate_up_quant(None, None, L["g"][0], L["g"][1], L["u"][0], L["u"][1], hq, hs,
                                     pro=fused.Producer.rmsnorm(hid, nw_post, 1e-6), level=1)
                ch.gemm_i8(hq, hs, L["d"][0], L["d"][1], hid, residual=hid, level=2)
                ch.proj3(None, None, L["qkv"][0], L["qkv"][1], L["z"][0], L["z"][1], None, None, qkvz,
                         pro=fused.Producer.rmsnorm(hid, nw_in, 1e-6, q=xq, s=xs), level=3)
                chains.append(ch.build())

            def run_chain():
                for ch in chains:
                    ch.run()

            chain_res[M] = timed(run_chain)
            if any(ch.wait_error() for ch in chains):
                raise RuntimeError("engine chain: a dependency wait gave up")
            log(f"engine {kind} layer with producers M={M:4d}: {chain_res[M] * 1e6:7.1f} us as one engine-chain "
                f"launch per layer")
    act_bytes = lambda M: M * (2048 * 3 + 6144) + M * 4 * (32 * 3 + 96)
    out_bytes = lambda M: M * 2 * (8192 + 2048 * 2 * 2) + M * (6144 + 96 * 4)
    dec_bytes = {M: layer_wbytes + act_bytes(M) + out_bytes(M) for M in (1, 4)}
    flops = 2 * 512 * (2048 * 8192 + 2048 * 2048 + 2048 * 12288 + 6144 * 2048)
    for M in ms:
        extra = (f"{dec_bytes[M] / res[M] / 1e9:7.0f} GB/s" if M in dec_bytes
                 else f"{flops / res[M] / 1e12:7.1f} TOPS")
        log(f"engine {kind} layer M={M:4d}: {res[M] * 1e6:8.1f} us per layer  {extra}")
    for M in (1, 4):
        log(f"engine {kind} layer chain M={M}: {dec_bytes[M] / chain_res[M] / 1e9:7.0f} GB/s")
    return dec_bytes, flops, res, pro_res, chain_res


def check_sweep(ctx, kind, shapes, head, ms, layers, max_cols=4096, every_layer_cols=None):
    """Checks the outputs the timed decode steps left: every shape of the last layer
    copy and sampled columns of the vocabulary head, at every M, against the fp32 CPU
    path (torch_dequant + fp32 matmul of the same fp16 activations).  With
    `every_layer_cols` set, the other layer copies are checked too, each job on that
    many sampled columns (the columns are picked on the device, so only they are
    copied and dequantized).  Returns the worst normalized error max|y - ref| /
    max|ref| and whether it is within the 2e-3 tolerance plus the fp16 output
    rounding (2**-11 relative)."""
    import torch
    lw, hw, xs, outs, hout = ctx[:5]
    worst = 0.0
    gen = torch.Generator().manual_seed(17)

    def pick(n, k):
        return torch.randperm(n, generator=gen)[:k].sort().values

    jobs = [(lw[layers - 1][i], layers - 1, i, None) for i in range(len(shapes))]
    if every_layer_cols:
        jobs += [(lw[l][i], l, i, pick(shapes[i][2], every_layer_cols))
                 for l in range(layers - 1) for i in range(len(shapes))]
    jobs.append((hw, None, None, pick(head[2], max_cols)))
    njobs = 0
    for w, l, i, cols in jobs:
        if cols is None:
            wd = torch_dequant(kind, w.w.cpu(), w.s.cpu())
        else:
            cd = cols.to(w.w.device)
            wd = torch_dequant(kind, w.w[:, cd].cpu(), (w.s[cd] if kind == "w8" else w.s[:, cd]).cpu())
        for M in ms:
            x = xs[M][:, :w.K].float().cpu()
            ref = x @ wd
            y = (outs[M][l][i] if l is not None else hout[M])
            y = (y if cols is None else y[:, cols.to(y.device)]).float().cpu()
            err = float((y - ref).abs().max() / ref.abs().max())
            worst = max(worst, err)
        njobs += 1
    what = f"every shape of layer copy {layers - 1}"
    if every_layer_cols:
        what += f", {every_layer_cols} sampled columns of every shape of layer copies 0-{layers - 2}"
    return {"max_rel_err": round(worst, 6), "ok": worst <= 2e-3 + 2.0 ** -11, "jobs": njobs,
            "checked": (f"{what} and {max_cols} sampled vocab-head columns, M={'/'.join(map(str, ms))}, "
                        "against dequantize + fp32 matmul on the CPU")}


# ------------------------------------------------------------------ CPU baseline

def _cpu_model() -> str:
    import subprocess
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def torch_dequant(kind, w, s):
    """The reference's CPU path for one weight (quant_formats.py:6-9): dequantize to
    fp32 with torch on the CPU.  W8: w[k, n] * s[n]; W4 g128: (nibble - 8) * s[k // 128, n]
    with the low nibble of packed byte (j, n) at k = 2j (w4.py:5-11)."""
    import torch
    if kind == "w8":
        return w.to(torch.float32) * s.to(torch.float32)[None, :]
    K2, N = w.shape
    nib = torch.stack((w & 15, w >> 4), dim=1).reshape(2 * K2, N)
    sc = s.to(torch.float32).repeat_interleave(2 * K2 // s.shape[0], dim=0)
    return (nib.to(torch.int16) - 8).to(torch.float32) * sc


def cpu_baseline(kind, shapes, head, budget_s=30.0):
    """The reference's CPU path on the decode workload at M = 1 (dequantize, then an
    fp32 matmul): for every layer shape and the whole vocabulary head, dequantize the
    weight to fp32 with torch, then torch.matmul in fp32, on the host's cores
    (torch.set_num_threads).  Dequantization and matmul are timed separately, each
    the median of 10 runs after 2 warm-ups; GB/s over the same algorithmic bytes as
    the GPU line.  The torch dequantization is first checked bit for bit against the
    oracle."""
    import numpy as np
    import torch
    if str(ROOT) not in sys.path:
        sys.path.insert(0, str(ROOT))
    from oracle import ref_cpu as R

    affinity = len(os.sched_getaffinity(0))
    threads = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity)))
    torch.set_num_threads(threads)
    gen = torch.Generator().manual_seed(5)
    sample = list(shapes) + [head]
    t_deq = t_mm = 0.0
    nbytes = 0
    rows = []
    t_start = time.perf_counter()
    for i, (name, K, N) in enumerate(sample):
        x = torch.randn((1, K), generator=gen).to(torch.float16)
        if kind == "w8":
            w = torch.randint(-127, 128, (K, N), generator=gen, dtype=torch.int8)
            s = ((torch.randn(N, generator=gen) * 0.02).abs() / 127).to(torch.float16)
            nbytes += bytes_w8(1, K, N)
        else:
            w = torch.randint(0, 256, (K // 2, N), generator=gen, dtype=torch.uint8)
            s = ((torch.randn((K // 128, N), generator=gen) * 0.02).abs() / 7).to(torch.float16)
            nbytes += bytes_w4(1, K, N)
        if i == 0:  # the timed path is the oracle's dequantization, bit for bit
            wd = torch_dequant(kind, w[:256], s if kind == "w8" else s[:4]).numpy()
            ref = (R.dequant_w8_f32(w[:256].numpy(), s.numpy()) if kind == "w8"
                   else R.dequant_w4_f32(w[:256].numpy(), s[:4].numpy()))
            if not np.array_equal(wd, ref):
                raise RuntimeError("cpu_baseline: torch dequantization differs from the oracle")
        deq, mm = [], []
        for rep in range(12):
            t0 = time.perf_counter()
            wd = torch_dequant(kind, w, s)
            t1 = time.perf_counter()
            y = torch.matmul(x.to(torch.float32), wd)
            t2 = time.perf_counter()
            if rep >= 2:
                deq.append(t1 - t0)
                mm.append(t2 - t1)
            del wd, y
        d, m = float(np.median(deq)), float(np.median(mm))
        t_deq += d
        t_mm += m
        rows.append((name, K, N, d, m))
        if time.perf_counter() - t_start > 4 * budget_s:
            break
    log("cpu baseline (" + kind + "): " + ", ".join(f"{n} {d * 1e3:.1f}+{m * 1e3:.1f} ms" for n, _, _, d, m in rows))
    return {
        "value": round(nbytes / (t_deq + t_mm) / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": _cpu_model(),
        "affinity_cpus": affinity,
        "dequant_s": round(t_deq, 5),
        "matmul_s": round(t_mm, 5),
        "sample": (f"M=1 decode of every layer shape and the whole vocab head ({kind}): torch on the CPU, "
                   f"dequantize to fp32 then fp32 torch.matmul, {threads} threads; per shape the median "
                   f"of 10 runs after 2 warm-ups, dequantization and matmul timed separately"),
    }


# ------------------------------------------------------------------ counter runs

def head_pmc(args):
    """For `rocprofv3 --pmc` runs: a few launches of the vocabulary-head GEMVs (W8
    and W4 g128, M=1) and, as the known-size calibration for the byte counters, a
    1 GiB device-to-device copy (torch's copy kernel: 1 GiB read, 1 GiB written)."""
    import torch
    dev = torch.device("cuda", 0)
    lin = importlib.import_module(f"{ALIAS}.kernels.linear")
    gen = torch.Generator().manual_seed(7)
    _, K, N = HEAD
    x = torch.randn((1, K), generator=gen).to(torch.float16).to(dev)
    out = torch.empty((1, N), dtype=torch.float16, device=dev)
    for kind in ("w8", "w4"):
        w = Weights(kind, K, N, dev, gen)
        for _ in range(args.steps):
            w.run(lin, x, out)
        del w
    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "head-pmc", "w8_bytes_per_launch": bytes_w8(1, K, N),
                      "w4_bytes_per_launch": bytes_w4(1, K, N), "copy_bytes": 1 << 30}), flush=True)
    return 0


def prefill_w4_cases(args):
    """For `rocprofv3` runs comparing the W4 and W8 prefill kernels: for each of the
    three M = 2048 prefill shapes (2048x6144, 6144x2048, 2048x2048), 3 eager launches of
    W8 (fp16 column scales), then 3 of W4 group 128 with fp16 scales, and on 2048x6144
    also 3 each with bf16 and fp32 group scales (random fp16 x)."""
    import torch
    dev = torch.device("cuda", 0)
    lin = importlib.import_module(f"{ALIAS}.kernels.linear")
    g = torch.Generator().manual_seed(3)
    M = 2048
    for (K, N) in [(2048, 6144), (6144, 2048), (2048, 2048)]:
        x = torch.randn(M, K, generator=g).to(torch.float16).to(dev)
        w8 = torch.randint(-127, 128, (K, N), generator=g, dtype=torch.int8).to(dev)
        s8 = (torch.rand(N, generator=g) * 1e-3).to(torch.float16).to(dev)
        p4 = torch.randint(0, 256, (K // 2, N), generator=g, dtype=torch.uint8).to(dev)
        s4 = (torch.rand(K // 128, N, generator=g) * 1e-3).to(torch.float16).to(dev)
        y = torch.empty(M, N, dtype=torch.float16, device=dev)
        for _ in range(3):
            lin.linear_w8(x, w8, s8, y)
        for _ in range(3):
            lin.linear_w4(x, p4, s4, y)
        if (K, N) == (2048, 6144):
            for dt in (torch.bfloat16, torch.float32):
                sx = s4.to(dt)
                for _ in range(3):
                    lin.linear_w4(x, p4, sx, y)
        torch.cuda.synchronize()
    print(json.dumps({"workload": "prefill-pmc", "cases": "w4"}), flush=True)
    return 0


def prefill_pmc(args):
    """For `rocprofv3 --pmc` runs: a few launches of the dominant prefill GEMM (W8,
    M=2048, K=2048, N=6144) and the same 1 GiB device copy as the calibration; with
    `--pmc-cases w4`, the W4 / W8 comparison of prefill_w4_cases instead."""
    import torch
    if args.pmc_cases == "w4":
        return prefill_w4_cases(args)
    dev = torch.device("cuda", 0)
    lin = importlib.import_module(f"{ALIAS}.kernels.linear")
    gen = torch.Generator().manual_seed(8)
    M, K, N = 2048, 2048, 6144
    w = Weights("w8", K, N, dev, gen)
    x = torch.randn((M, K), generator=gen).to(torch.float16).to(dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    for _ in range(args.steps):
        w.run(lin, x, out)
    a = torch.empty(1 << 30, dtype=torch.uint8, device=dev)
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "prefill-pmc", "flops_per_launch": 2 * M * K * N,
                      "algorithmic_bytes": K * N + 2 * N + 2 * M * K + 2 * M * N, "copy_bytes": 1 << 30}),
          flush=True)
    return 0


def decode_pmc(args):
    """For `rocprofv3 --pmc` runs: `--steps` launches of the decode chain of
    `--pmc-kind` weights (every linear of 8 layer copies of the 2B-class layer, plus the
    vocab head unless `--head own` gives it a launch of its own, M = 1, dependency
    levels per `--levels`) and the same 1 GiB device copy as the calibration of the
    byte counters."""
    import torch
    args.launch = "chain"
    total, step, ev, step_bytes, record, ctx = decode_sweep(args, args.pmc_kind, LAYER_SHAPES, HEAD, [1], args.layers)
    for _ in range(args.steps):
        step()
    a = torch.empty(1 << 30, dtype=torch.uint8, device=torch.device("cuda", 0))
    b = torch.empty_like(a)
    for _ in range(2):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "decode-pmc", "kind": args.pmc_kind, "head": args.head,
                      "levels": args.levels, "bytes_per_launch": step_bytes[1],
                      "copy_bytes": 1 << 30}), flush=True)
    return 0


def layout_bench(args):
    """The load-time layout producers at a 9B-class projection (K=4096, N=12288):
    GPU requantization of fp32 weights (W8 per column, W4 g32) and the GPTQ / AWQ int4
    repacks (GPTQ, AWQ, compressed-tensors).  HBM-bound byte work: algorithmic bytes = one read of the input and one
    write of the outputs; time per launch from HIP events on the launching stream."""
    import torch
    dev = torch.device("cuda", 0)
    lay = importlib.import_module(f"{ALIAS}.kernels.layout")
    gen = torch.Generator().manual_seed(9)
    K, N = 4096, 12288
    w = (torch.randn((K, N), generator=gen) * 0.02).to(dev)
    qg = torch.randint(-2 ** 31, 2 ** 31 - 1, (K // 8, N), generator=gen, dtype=torch.int32).to(dev)
    qa = torch.randint(-2 ** 31, 2 ** 31 - 1, (K, N // 8), generator=gen, dtype=torch.int32).to(dev)
    qc = torch.randint(-2 ** 31, 2 ** 31 - 1, (N, K // 8), generator=gen, dtype=torch.int32).to(dev)
    cases = {
        "requant_w8_row": (lambda: lay.requant_w8_row(w), 4 * K * N + K * N + 4 * N),
        "requant_w4_sym_g32": (lambda: lay.requant_w4_sym(w, 32), 4 * K * N + K * N // 2 + 2 * (K // 32) * N),
        "w4_repack_gptq": (lambda: lay.gptq_w4_to_engine(qg), K * N // 2 + K * N // 2),
        "w4_repack_awq": (lambda: lay.awq_w4_to_engine(qa), K * N // 2 + K * N // 2),
        "w4_repack_ct": (lambda: lay.ct_w4_to_engine(qc, K=K), K * N // 2 + K * N // 2),
    }
    res = {}
    for name, (fn, nbytes) in cases.items():
        for _ in range(args.warmup):
            fn()
        st = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(st)
        for _ in range(args.steps):
            fn()
        e1.record(st)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.steps
        res[name] = {"us": round(us, 2), "bytes": nbytes, "GB/s": round(nbytes / us / 1e3, 1),
                     "frac_of_8TB/s": round(nbytes / us / 1e3 / 8000.0, 3)}
    line = {"metric": "layout producers, HBM GB/s", "value": res["requant_w8_row"]["GB/s"], "unit": "GB/s",
            "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
            "data": "synthetic (seeded random fp32 weights and int32 words)", "dtype": "f32 / u8 / i32",
            "config": {"workload": "layout producers at K=4096, N=12288", "kernels": res}}
    print(json.dumps(line), flush=True)
    return 0


# ------------------------------------------------------------------ main

def read_traffic(kernel_tag):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3 --pmc
    summaries (profiles/*_hbm_traffic.md: FETCH_SIZE and WRITE_SIZE, each scaled by
    the reading of a known-size copy), or None."""
    lines = []
    for p in sorted((ROOT / "profiles").glob("*_hbm_traffic.md")):
        lines += p.read_text().splitlines()
    for line in lines:
        if line.startswith(f"traffic_bytes_per_launch[{kernel_tag}]"):
            try:
                return int(line.split("=")[1].split()[0])
            except (IndexError, ValueError):
                return None
    return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--workload", default="decode-w8",
                    choices=["decode-w8", "decode-w4", "prefill", "chain-w4", "single", "head-pmc",
                             "prefill-pmc", "decode-pmc", "engine-w8", "engine-w4", "layout", "prefill-9b"])
    ap.add_argument("--layers", type=int, default=8)
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--launch", default="chain", choices=["chain", "graph"],
                    help="decode workloads: one persistent chain launch per M, or one launch per GEMV "
                         "replayed as a HIP graph")
    ap.add_argument("--levels", default=None, choices=["layer", "flat"],
                    help="chain dependency levels: per decode layer, or all independent (default: flat for "
                         "the decode sweeps, whose shapes are independent; layer for the 9B-class decode chain)")
    ap.add_argument("--head", default=None, choices=["chain", "own"],
                    help="chain launches: the vocabulary head inside the chain launch, or as its own launch "
                         "(the wide GEMV plan) after it (default: own for the 9B-class W4 chain, chain "
                         "otherwise, whichever measured faster)")
    ap.add_argument("--pmc-kind", default="w8", choices=["w8", "w4"], help="decode-pmc: weight format")
    ap.add_argument("--pmc-cases", default="dominant", choices=["dominant", "w4"],
                    help="prefill-pmc: the dominant W8 GEMM, or the W4 / W8 comparison on the three shapes")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--detail", action="store_true", help="per-shape table on stderr")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU (the path has no multi-GPU part); "
              "run it with --gpus 1", file=sys.stderr)
        return 2

    import torch
    _load_package()
    from qwen35_amd.kernels import qlin
    qlin.lib()
    if not torch.cuda.is_available():
        print("bench.py: no GPU", file=sys.stderr)
        return 1

    wl = args.workload
    if args.head is None:
        args.head = "own" if wl == "chain-w4" else "chain"
    if wl == "head-pmc":
        return head_pmc(args)
    if wl == "prefill-pmc":
        return prefill_pmc(args)
    if wl == "decode-pmc":
        return decode_pmc(args)
    if wl == "layout":
        return layout_bench(args)
    ms = [1, 2, 4]
    roof = None
    if args.no_graph:
        args.launch = "graph"
    if args.levels is None:
        args.levels = "layer" if args.workload == "chain-w4" else "flat"
    if wl in ("decode-w8", "decode-w4", "chain-w4", "single"):
        kind = "w4" if wl in ("decode-w4", "chain-w4") else "w8"
        if wl == "chain-w4":
            shapes, head, layers, ms = CHAIN_SHAPES, CHAIN_HEAD, 32, [1, 4]
        elif wl == "single":
            shapes, head, layers, ms = [], ("gate", 2048, 6144), 0, [1]
        else:
            shapes, head, layers = LAYER_SHAPES, HEAD, args.layers
        if wl == "single":
            args.launch = "graph"
        total, step, head_ev, head_bytes, record, ctx = decode_sweep(args, kind, shapes, head, ms, layers)
        period_timing = args.launch == "chain" and args.head == "chain"
        if period_timing:
            # the step is nothing but the chain launches (one per M): the timed steps hold
            # no event but one pair bracketing them (an event recorded between launches
            # costs the step 8-11 us per launch, measured), and the chain's average launch
            # period -- the bracket over the launches, gaps between launches included, so
            # at least the kernel's duration -- prices the roofline.  (With the vocab head
            # as its own launch after each chain, events around each chain launch do.)
            span = {}
            t = time_steps(step, args.steps, args.warmup, None, span)
            period = span["ms"] * 1e-3 / (args.steps * len(ms))
            durs = [(M, period) for M in ms]
            # per-M launch times for the log: a short pass with events around each launch
            time_steps(step, 5, 0, record)
        else:
            t = time_steps(step, args.steps, args.warmup, record)
            # the dominant kernel (with per-GEMV launches the vocabulary-head GEMV; with a
            # chain followed by the head's own launch the chain), every launch of the
            # timed steps timed live with HIP events on its launch stream
            durs = [(M, e0.elapsed_time(e1) * 1e-3) for M in ms for (e0, e1) in head_ev[M]]
        value = total / t / 1e9
        dur = sum(d for _, d in durs) / len(durs)
        hb = sum(head_bytes[M] for M, _ in durs) / len(durs)
        achieved = hb / dur / 1e9
        if args.launch == "chain":
            tag = f"chain-{kind}-{wl}"
            kname = (f"chain_kernel {kind}: {layers} layer copies x {len(shapes)} linears"
                     + (f" + vocab head {head[1]}x{head[2]}" if args.head == "chain" else "")
                     + f", {args.levels} levels, M={'/'.join(map(str, ms))}")
            if args.head == "own":
                tag += "-layers"
        else:
            tag = f"{kind}-{head[1]}x{head[2]}"
            kname = f"skinny_kernel {kind} vocab head {head[1]}x{head[2]}, M={'/'.join(map(str, ms))}"
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": read_traffic(tag),
                "kernel": kname, "bytes_per_launch": int(hb), "avg_launch_us": round(dur * 1e6, 2)}
        if args.detail and args.launch != "chain":
            detail_table(ctx, kind, shapes, head, ms)
        per_m = {M: sum(e0.elapsed_time(e1) for e0, e1 in head_ev[M]) / len(head_ev[M]) for M in ms}
        if period_timing:
            roof["timing"] = ("average launch period: one HIP event pair bracketing the timed steps, "
                              "divided by the launches in them (gaps between launches included)")
            roof["event_us_by_M"] = {str(M): round(v * 1e3, 1) for M, v in per_m.items()}
        else:
            roof["timing"] = "HIP events around every launch of the kernel in the timed steps"
        log(("chain" if args.launch == "chain" else "vocab head") + " per-launch us by M: " +
            ", ".join(f"M={M}: {v * 1e3:.1f} ({head_bytes[M] / v / 1e6:.0f} GB/s)" for M, v in per_m.items()))
        other = None
        check = None
        if layers > 0:
            # the outputs the timed steps left, before any other run rewrites them; the
            # 9B-class chain is checked on every layer copy (sampled columns)
            check = check_sweep(ctx, kind, shapes, head, ms, layers,
                                every_layer_cols=256 if wl == "chain-w4" else None)
            log(f"output check: {check}")
            if not check["ok"]:
                print(json.dumps({"error": "decode sweep outputs out of tolerance", **check}))
                return 1
        if args.launch == "chain":
            for M, ch in ctx[6].items():
                if ch.wait_error():
                    log(f"chain M={M}: a dependency wait gave up")
                    return 1
            # the same step with the other dependency structure, for comparison
            main_levels = args.levels
            args.levels = "flat" if main_levels == "layer" else "layer"
            tot2, step2, ev2, sb2, rec2, ctx2 = decode_sweep(args, kind, shapes, head, ms, layers, reuse=ctx)
            t2 = time_steps(step2, max(3, args.steps // 2), 2)
            other = {"levels": args.levels, "GB_per_s": round(tot2 / t2 / 1e9, 1),
                     "ms_per_step": round(t2 * 1e3, 4)}
            log(f"same step with {args.levels} levels: {tot2 / t2 / 1e9:.0f} GB/s")
            args.levels = main_levels
            del ctx2
        unit = "GB/s"
        config = {"workload": {"decode-w8": "int8 decode GEMV sweep, 2B-class layer shapes + vocab head",
                               "decode-w4": "W4 g128 decode GEMV sweep, 2B-class layer shapes + vocab head",
                               "chain-w4": "9B-class W4 g128 decode chain: 32 layers + vocab head",
                               "single": "single int8 linear 2048x6144"}[wl],
                  "rows_M": ms, "layer_copies": layers,
                  "shapes_KN": [[K, N] for (_, K, N) in shapes] + [[head[1], head[2]]],
                  "bytes_per_step": total,
                  "launch": ({"chain": f"one persistent chain launch per M ({args.levels} dependency levels)"
                                       + ("" if args.head == "chain" else ", then the vocab head as its own launch"),
                              "graph": "hipgraph per M for layer shapes, eager vocab head"}[args.launch]
                             if not args.no_graph else "eager")}
        if other is not None:
            config["other_levels"] = other
        if check is not None:
            config["output_check"] = check
        if wl in ("decode-w8", "decode-w4"):
            # beside the sweep: the call sequence the engine's decode step makes, the
            # four engine-signature linears of one layer (int8 codes + per-64 scales),
            # as four launches per layer and as one engine-chain launch per layer
            # that also makes the activations (its producers)
            dec_bytes, _, res, pro_res, chain_res = engine_bench(args, kind, ms=(1, 4))
            config["engine_signature"] = {
                "layer_calls": "proj3, gemm_i8 + residual, mlp_gate_up_quant, gemm_i8 + residual "
                               "(one 2B-class layer, hipgraph of all layer copies per M)",
                "bytes_per_layer": {str(M): dec_bytes[M] for M in (1, 4)},
                "calls_us_per_layer": {str(M): round(res[M] * 1e6, 1) for M in (1, 4)},
                "calls_frac": {str(M): round(dec_bytes[M] / res[M] / 1e9 / HBM_PEAK_GBS, 4) for M in (1, 4)},
                "chain_with_producers_us_per_layer": {str(M): round(chain_res[M] * 1e6, 1) for M in (1, 4)},
                "chain_frac": {str(M): round(dec_bytes[M] / chain_res[M] / 1e9 / HBM_PEAK_GBS, 4)
                               for M in (1, 4)},
                "calls_with_producers_us_per_layer": {str(M): round(pro_res[M][1] * 1e6, 1) for M in (1, 4)}}
        dtype = "f16 x int8" if kind == "w8" else "f16 x int4"
    elif wl in ("engine-w8", "engine-w4"):
        kind = wl.split("-")[1]
        dec_bytes, pf_flops, res, pro_res, chain_res = engine_bench(args, kind)
        # value: decode rows M = 1 and 4 through the engine's calls, weight-streaming GB/s
        t = (res[1] + res[4]) / 2
        value = (dec_bytes[1] + dec_bytes[4]) / (res[1] + res[4]) / 1e9
        unit = "GB/s"
        config = {"workload": f"engine-signature calls of one 2B-class layer ({kind}): proj3, gemm_i8 + "
                              "residual, mlp_gate_up_quant, gemm_i8 + residual",
                  "rows_M": [1, 4], "layer_copies": args.layers,
                  "shapes_KN": [[K, N] for (_, K, N) in ENGINE_LAYER],
                  "prefill_chunk_M512_us_per_layer": round(res[512] * 1e6, 1),
                  "prefill_chunk_M512_tops": round(pf_flops / res[512] / 1e12, 1),
                  "with_producers_us_per_layer": {
                      str(M): {"producer_then_linear": round(u * 1e6, 1), "fused": round(f * 1e6, 1),
                               **({"engine_chain": round(chain_res[M] * 1e6, 1)} if M in chain_res else {})}
                      for M, (u, f) in pro_res.items()},
                  "engine_chain_GB_per_s": {str(M): round(dec_bytes[M] / chain_res[M] / 1e9, 1) for M in (1, 4)},
                  "launch": "hipgraph of all layers per M"}
        dtype = "i8 x int8" if kind == "w8" else "i8 x int4"
    else:
        shapes = PREFILL_SHAPES_9B if wl == "prefill-9b" else PREFILL_SHAPES
        flops, t, roof, nsets = prefill_bench(args, shapes)
        value = flops / t / 1e12
        unit = "TFLOP/s"
        config = {"workload": "prefill GEMM, int8 and W4 g128, M in 128/512/2048" +
                              (", 9B-class layer shapes" if wl == "prefill-9b" else ""),
                  "shapes_KN": [[K, N] for (_, K, N) in shapes], "flops_per_step": flops,
                  "weight_copy_sets": nsets,
                  "launch": "hipgraph per copy set for 17 cases, eager dominant case"}
        dtype = "f16 x int8/int4"

    cpu = None
    if not args.no_cpu_baseline and wl in ("decode-w8", "decode-w4"):
        cpu = cpu_baseline("w8" if wl == "decode-w8" else "w4", LAYER_SHAPES, HEAD, args.cpu_seconds)

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": unit, "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(t * 1e3, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded random weights in the engine layouts)", "config": config,
        "roofline": roof, "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
