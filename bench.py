"""Benchmark of the MI355X quantized compute path (one GPU).

Headline: batch-1 decode GEMV at the FFN shapes,
Q4_K 14336x4096 (up/gate) and 4096x14336 (down). One step = quantize the
activation (per-256, as the reference's matmul_q4_k does) + GEMV, for both
shapes (one launch each: the GEMV quantizes its fp32 activation in-kernel),
on weight copies rotated so that the working set (>= 512 MB) exceeds the
256 MB Infinity Cache and every weight byte comes from HBM. Inputs are
resident in HBM before timing. value = algorithmic bytes per step / step time.

Also reported under "extra": the Q4_0 and Q8_0 GEMVs (configs 1-2), the Q6_K
GEMV, each with its kernel-only bandwidth; the prefill GEMMs (config 3); the
decode attention and the decoder layer (config 4); the MoE expert FFN
(config 5); the prefill attention and the decoder layer over a 512-token
prompt chunk (config 4's layer, the prefill path); the output head of a
128256-token vocabulary with the device top-k and draw.

`roofline` is the dominant kernel (Q4_K GEMV, up shape): algorithmic bytes per
launch / average launch duration, from HIP events around back-to-back launches
on the stream the kernels run on, captured in a HIP graph so host launch
overhead is not counted. `cpu_baseline` times the reference engine's
own matmul_q4_k (oracle/_ref, compiled from the reference sources) on the
host, over a bounded sample; `cpu_baseline.rows` times its matmul_batch,
attention_prefill_q8 and matmul_q6_k on the prefill GEMM, prefill attention
and output-head shapes.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--only NAME] [--no-cpu]

--only runs one line N times for a profiler: a GEMV shape (q4k_up, ...),
step (the headline step), copy, gemm_*, layer, moe, attn, head,
attn_prefill, layer_prefill.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0  # dense MFMA, MI355X
INT8_PEAK_TOPS = 5000.0
METRIC = "Q4_K/Q8_0 GEMV HBM GB/s (% of peak); prefill GEMM TFLOPS (% MFMA peak)"
ROTATE_BYTES = 640 << 20  # >= 2x the 256 MB Infinity Cache


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_kernel_bytes(qtype, rows, cols):
    """Algorithmic HBM bytes of one GEMV launch: the GGUF weight bytes, the
    quantized activation (int8 + fp32 scale + int32 sum per 32) and y (fp32)."""
    from desireeia_amd import synth
    return rows * synth.row_bytes(qtype, cols) + cols + cols // 32 * 8 + rows * 4


def step_bytes(qtype, rows, cols):
    """Algorithmic bytes of one quantize+GEMV step: weights + x fp32 + y fp32
    (the per-call figure of the benchmark plan)."""
    from desireeia_amd import synth
    return rows * synth.row_bytes(qtype, cols) + cols * 4 + rows * 4


class GemvCase:
    def __init__(self, qtype, rows, cols, seed, dev):
        import torch
        from desireeia_amd import ops, synth
        self.qtype, self.rows, self.cols = qtype, rows, cols
        w = synth.gen_weights(qtype, rows, cols, seed)
        m0 = ops.QuantMatrix.from_gguf(qtype, w, rows, cols, device=dev)
        ncopy = max(2, -(-ROTATE_BYTES // m0.buf.numel()))
        self.mats = [m0] + [m0.clone() for _ in range(ncopy - 1)]
        self.x = torch.from_numpy(synth.gen_act(cols, seed + 1)).to(dev)
        self.kind = ops.act_kind_for(m0.fmt)
        self.act = ops.quantize_act(self.x, self.kind)
        self.y = torch.empty(rows, dtype=torch.float32, device=dev)
        self.i = 0

    def step(self):
        # quantize + GEMV: one launch, the activation quantized in-kernel
        from desireeia_amd import ops
        m = self.mats[self.i]
        self.i = (self.i + 1) % len(self.mats)
        ops.matmul(m, self.x, out=self.y)

    def kernel(self):
        from desireeia_amd import ops
        m = self.mats[self.i]
        self.i = (self.i + 1) % len(self.mats)
        ops.gemv(m, self.act, out=self.y)


class GemmCase:
    """Prefill GEMM (config 3): X [n_tok][cols] fp32 -> Y [n_tok][rows]."""

    def __init__(self, qtype, rows, cols, n_tok, seed, dev, tiles=False):
        import torch
        from desireeia_amd import ops, synth
        self.qtype, self.rows, self.cols, self.n_tok = qtype, rows, cols, n_tok
        w = synth.gen_weights(qtype, rows, cols, seed)
        m0 = ops.QuantMatrix.from_gguf(qtype, w, rows, cols, device=dev)
        self.mats = [m0, m0.clone()]
        if tiles:  # the opt-in tile copies (dq_gemm_tiles_pack) in place of the packed rows
            self.mats = [ops.GemmTiles(m) for m in self.mats]
        self.x = torch.from_numpy(synth.gen_act((n_tok, cols), seed + 1)).to(dev)
        self.work = ops.gemm_workspace(m0, n_tok)
        self.y = torch.empty(n_tok, rows, dtype=torch.float32, device=dev)
        self.i = 0
        ops.gemm(m0, self.x, out=self.y, work=self.work)

    def step(self):
        from desireeia_amd import ops
        m = self.mats[self.i]
        self.i ^= 1
        ops.gemm(m, self.x, out=self.y, work=self.work)

    def kernel(self):
        from desireeia_amd import _lib, ops
        m = self.mats[self.i]
        self.i ^= 1
        lib = _lib.load()
        _lib.check(lib.dq_gemm_f16act(m.fmt, ops._ptr(m.buf), m.rows, m.cols, ops._ptr(self.work), self.n_tok,
                                      ops._ptr(self.y), ops._stream()), "dq_gemm_f16act")

    def flops(self):
        return 2.0 * self.n_tok * self.rows * self.cols


LAYER_WEIGHT_BYTES = 138903552   # config 4 Q4_K_M layer, GGUF bytes
KV_READ_BYTES = 4097 * 8 * 136 * 2  # K and V rows of positions 0..4096


class LayerCase:
    """Config 4: Llama-style decoder layer (hidden 4096, 32/8 heads of 128,
    FFN 14336, Q4_K_M mix) at position 4096 over a Q8_0 KV cache of 4096
    prior N(0,1) tokens. n_layers distinct layers (weights copied, so every
    byte comes from HBM) are chained like a model's layers; the position is a
    device value, so the chain is one replayable graph."""

    def __init__(self, dev, n_layers=4, pos=4096, seed=40):
        import torch
        from desireeia_amd import ops, synth
        E, H, KV, HD, F = 4096, 32, 8, 128, 14336
        shapes = {"q": (synth.Q4_K, H * HD, E), "k": (synth.Q4_K, KV * HD, E), "v": (synth.Q6_K, KV * HD, E),
                  "o": (synth.Q4_K, E, H * HD), "gate": (synth.Q4_K, F, E), "up": (synth.Q4_K, F, E),
                  "down": (synth.Q6_K, E, F)}
        base = {nm: ops.QuantMatrix.from_gguf(qt, synth.gen_weights(qt, r, c, seed + i), r, c, device=dev)
                for i, (nm, (qt, r, c)) in enumerate(shapes.items())}
        rng = np.random.default_rng(seed)
        self.pos, self.n_ctx = pos, pos + 1
        self.dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        self.layers = []
        for li in range(n_layers):
            mats = base if li == 0 else {nm: m.clone() for nm, m in base.items()}
            an = torch.from_numpy((1 + 0.02 * rng.standard_normal(E)).astype(np.float32))
            fn = torch.from_numpy((1 + 0.02 * rng.standard_normal(E)).astype(np.float32))
            L = ops.DecoderLayer(mats, an, fn, H, KV, HD, self.n_ctx, device=dev)
            L.set_rope(pos)
            kv = torch.randn(pos, 2, KV * HD, device=dev, generator=torch.Generator(device=dev).manual_seed(li))
            for p in range(pos):
                L.cache.write(kv[p, 0], kv[p, 1], p)
            self.layers.append(L)
        self.x = torch.from_numpy(synth.gen_act(E, seed + 99)).to(dev)
        self.bufs = [torch.empty(E, dtype=torch.float32, device=dev) for _ in range(2)]
        torch.cuda.synchronize()

    def step(self):
        x = self.x
        for i, L in enumerate(self.layers):
            y = self.bufs[i % 2]
            L.decode(x, self.dpos, out=y)
            x = y

    def bytes_per_layer(self):
        E, QD, F = 4096, 4096, 14336
        # weights + KV rows read + the new KV row written + x in / out
        return LAYER_WEIGHT_BYTES + KV_READ_BYTES + 2 * 1088 + 2 * E * 4


class AttnCase:
    """Decode attention alone at config 4's shape (32 query heads over 8 KV
    heads of 128, positions 0..4096), caches rotated over >= 640 MB."""

    def __init__(self, dev, pos=4096):
        import torch
        from desireeia_amd import ops
        self.pos = pos
        c0 = ops.KVCache(pos + 1, 8, 128, device=dev)
        kv = torch.randn(pos + 1, 2, 1024, device=dev, generator=torch.Generator(device=dev).manual_seed(7))
        for p in range(pos + 1):
            c0.write(kv[p, 0], kv[p, 1], p)
        ncopy = max(2, -(-ROTATE_BYTES // (2 * c0.k.numel())))
        self.caches = [c0]
        for _ in range(ncopy - 1):
            c = ops.KVCache(pos + 1, 8, 128, device=dev)
            c.k.copy_(c0.k)
            c.v.copy_(c0.v)
            self.caches.append(c)
        self.q = torch.randn(32 * 128, device=dev)
        self.out = torch.empty(32 * 128, device=dev)
        self.work = ops.attn_workspace(32, 8, 128, pos + 1, dev)
        self.i = 0

    def kernel(self):
        from desireeia_amd import ops
        c = self.caches[self.i]
        self.i = (self.i + 1) % len(self.caches)
        ops.attention_decode(self.q, c, 32, self.pos, out=self.out, work=self.work)


MOE_WEIGHT_BYTES = 8 * 99090432  # config 5: 8 experts x (gate, up, down) Q4_K


class MoeCase:
    """Config 5: MoE expert FFN, 8 experts top-2 (renormalised softmax), hidden
    4096, expert FFN 14336 (SwiGLU), Q4_K experts, 64 tokens of N(0,1); router
    logits N(0,1). The 792 MB of expert weights are 3x the Infinity Cache, so
    every call streams them from HBM."""

    def __init__(self, dev, n_tok=64, seed=50):
        import torch
        from desireeia_amd import ops, synth
        E, F, X = 4096, 14336, 8
        mk = lambda r, c, sd: ops.QuantMatrix.from_gguf(synth.Q4_K, synth.gen_weights(synth.Q4_K, r, c, sd), r, c,
                                                        device=dev)
        # the layer keeps the expert-tile copies only; the packed rows are freed here
        self.moe = ops.MoeLayer(mk(X * F, E, seed), mk(X * F, E, seed + 1), mk(X * E, F, seed + 2), n_expert=X,
                                n_expert_used=2)
        self.n_tok = n_tok
        self.x = torch.from_numpy(synth.gen_act((n_tok, E), seed + 3)).to(dev)
        self.lg = torch.from_numpy(synth.gen_act((n_tok, X), seed + 4)).to(dev)
        self.out = torch.empty(n_tok, E, dtype=torch.float32, device=dev)
        self.moe(self.x, self.lg, out=self.out)
        torch.cuda.synchronize()

    def step(self):
        self.moe(self.x, self.lg, out=self.out)

    def bytes(self):
        return MOE_WEIGHT_BYTES + self.n_tok * 4096 * 4 * 2 + self.n_tok * 8 * 4


class AttnPrefillCase:
    """Prefill attention at config 4's head shape (32 query heads over 8 KV
    heads of 128): n_tok prompt tokens after pos0 cached positions, every
    token attending causally to all earlier positions. Algorithmic work: the
    two products, 4 * hd flops per (row, key) pair."""

    def __init__(self, dev, pos0=3584, n_tok=512):
        import torch
        from desireeia_amd import ops
        self.pos0, self.n_tok = pos0, n_tok
        g = torch.Generator(device=dev).manual_seed(9)
        self.cache = ops.KVCache(pos0 + n_tok, 8, 128, device=dev)
        self.cache.write_batch(torch.randn(pos0 + n_tok, 1024, device=dev, generator=g),
                               torch.randn(pos0 + n_tok, 1024, device=dev, generator=g), 0)
        self.q = torch.randn(n_tok, 32 * 128, device=dev, generator=g)
        self.out = torch.empty_like(self.q)
        torch.cuda.synchronize()

    def kernel(self):
        from desireeia_amd import ops
        ops.attention_prefill(self.q, self.cache, 32, self.pos0, out=self.out)

    def flops(self):
        keys = self.n_tok * (self.pos0 + 1) + self.n_tok * (self.n_tok - 1) // 2
        return 4.0 * 128 * 32 * keys


class LayerPrefillCase:
    """Config 4's decoder layer (hidden 4096, 32/8 heads of 128, FFN 14336,
    Q4_K_M mix) over a prompt chunk of n_tok tokens at positions pos0..
    (dq_layer_prefill: seven prefill GEMMs, batched RoPE + KV rows, prefill
    attention, norms, SiLU, residuals). RMSNorm weights 0.25 / sqrt(4096) and
    0.3 / sqrt(4096) keep the synthetic activations O(1)."""

    def __init__(self, dev, pos0=0, n_tok=512, seed=60, tiles=False):
        import torch
        from desireeia_amd import ops, synth
        E, H, KV, HD, F = 4096, 32, 8, 128, 14336
        shapes = {"q": (synth.Q4_K, H * HD, E), "k": (synth.Q4_K, KV * HD, E), "v": (synth.Q6_K, KV * HD, E),
                  "o": (synth.Q4_K, E, H * HD), "gate": (synth.Q4_K, F, E), "up": (synth.Q4_K, F, E),
                  "down": (synth.Q6_K, E, F)}
        mats = {nm: ops.QuantMatrix.from_gguf(qt, synth.gen_weights(qt, r, c, seed + i), r, c, device=dev)
                for i, (nm, (qt, r, c)) in enumerate(shapes.items())}
        an, fn = torch.full((E,), 0.25 / 64), torch.full((E,), 0.3 / 64)
        self.layer = ops.DecoderLayer(mats, an, fn, H, KV, HD, pos0 + n_tok, device=dev)
        if tiles:  # the products read tile copies of the matrices (dq_gemm_tiles_pack)
            self.layer.use_gemm_tiles()
        g = torch.Generator(device=dev).manual_seed(seed)
        if pos0:
            self.layer.cache.write_batch(torch.randn(pos0, KV * HD, device=dev, generator=g),
                                         torch.randn(pos0, KV * HD, device=dev, generator=g), 0)
        self.pos0, self.n_tok = pos0, n_tok
        self.x = torch.randn(n_tok, E, device=dev, generator=g)
        self.out = torch.empty_like(self.x)
        self.rope = torch.stack([ops.rope_cache(HD, pos0 + t, 500000.0) for t in range(n_tok)]).to(dev)
        self.work = self.layer.prefill_workspace(n_tok)
        torch.cuda.synchronize()

    def step(self):
        self.layer.prefill(self.x, self.pos0, out=self.out, work=self.work, rope=self.rope)

    def flops(self):
        E, QD, KVD, F = 4096, 4096, 1024, 14336
        gemm = 2.0 * self.n_tok * (QD * E + 2 * KVD * E + E * QD + 3 * F * E)
        keys = self.n_tok * (self.pos0 + 1) + self.n_tok * (self.n_tok - 1) // 2
        return gemm + 4.0 * 128 * 32 * keys


class HeadCase:
    """Output head of a 128256-token vocabulary over hidden 4096 (Q6_K, as
    Llama-3 GGUF heads are commonly stored): final RMSNorm + head GEMV for one
    decoded token, then the top-40 and the draw (temperature 0.8, top-k 40,
    top-p 0.95, repeat penalty over 64 tokens) on the device."""

    def __init__(self, dev, rows=128256, cols=4096, seed=70):
        import torch
        from desireeia_amd import _lib, ops, synth
        self.rows, self.cols = rows, cols
        self.mat = ops.QuantMatrix.from_gguf(synth.Q6_K, synth.gen_weights(synth.Q6_K, rows, cols, seed), rows, cols,
                                             device=dev)
        self.x = torch.from_numpy(synth.gen_act(cols, seed + 1)).to(dev)
        self.norm = torch.ones(cols, device=dev)
        self.logits = torch.empty(rows, device=dev)
        self.sampler = ops.DeviceSampler(dev, hist=list(range(64)))
        a = _lib.CudaSampleArgs()
        a.temperature, a.top_k, a.top_p, a.penalty_repeat, a.penalty_last_n = 0.8, 40, 0.95, 1.1, 64
        a.kk, a.u = 104, 0.5
        self.args = a
        torch.cuda.synchronize()

    def logits_step(self):
        from desireeia_amd import ops
        ops.head_logits(self.mat, self.x, self.norm, out=self.logits)

    def select_step(self):
        from desireeia_amd import ops
        ids, vals = ops.topk(self.logits, 104)
        self.sampler.sample(ids, vals, self.args)

    def bytes(self):
        from desireeia_amd import synth
        # the weights (431 MB: more than the Infinity Cache, streamed each
        # call), x, the norm weights and the logits
        return gemv_kernel_bytes(synth.Q6_K, self.rows, self.cols) + 2 * self.cols * 4


def graph_time(fn, calls_per_graph, reps, warmup_reps=2):
    """Captures calls_per_graph calls of fn into one HIP graph and times `reps`
    replays with HIP events on the capturing stream. Returns us per call."""
    ts = replay_times(fn, calls_per_graph, reps, warmup_reps)
    return sum(ts) / len(ts)


WARMUP_MS = 25.0  # untimed graph replays before every timed set: the first few ms of a
                  # workload after set-up run up to 15% slower than its steady state


def replay_times(fn, calls_per_graph, reps, warmup_reps=2):
    """Captures calls_per_graph calls of fn into one HIP graph and times each
    of `reps` replays on its own (HIP events on the capturing stream, the
    stream the kernels run on), after warmup_reps untimed replays and at least
    WARMUP_MS of them. Returns us per call, one figure per replay."""
    import torch
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(calls_per_graph):
            fn()
    t0 = time.perf_counter()
    n = 0
    while n < warmup_reps or (time.perf_counter() - t0) * 1e3 < WARMUP_MS:
        g.replay()
        n += 1
        if n % 4 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
    ev[0].record()
    for i in range(reps):
        g.replay()
        ev[i + 1].record()
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) / calls_per_graph * 1e3 for i in range(reps)]


def kernel_stats(case, launches=400, fp32=False):
    """Average GEMV launch duration (us) over a graph of back-to-back launches
    on the rotated weight copies: the pre-quantized GEMV (dq_gemv), or with
    fp32=True the launch the benchmark step runs (dq_gemv_f32: the
    activation quantized in-kernel). Returns (us, GB/s of that launch's
    algorithmic bytes)."""
    per = 2 * len(case.mats)
    us = graph_time(case.step if fp32 else case.kernel, per, max(1, launches // per))
    b = (step_bytes if fp32 else gemv_kernel_bytes)(case.qtype, case.rows, case.cols)
    return us, b / us / 1e3


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemv_q4k_down_4096x14336_fp32_traffic.md")


def recorded_traffic():
    """HBM bytes per launch of the dominant kernel, from the FETCH_SIZE and
    WRITE_SIZE counter passes summarised in profiles/ (rocprofv3 cannot run
    inside this process; the file gives the commands). None if absent."""
    try:
        for line in open(TRAFFIC_FILE):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":")[1])
    except OSError:
        pass
    return None


def stream_read_ceiling(dev, nbytes, reps=20):
    """The device's streaming-read rate at one GEMV's size: dq_stream_read of
    nbytes (rounded up to 16 KB) over buffers rotated across >= 640 MB (every
    byte from HBM), one launch per call in a graph, over 4, 8 and 16 KB in
    flight per wave and 4, 8 and 16 waves per CU. Returns {"waves/CU x KB":
    GB/s} and the best."""
    import torch
    from desireeia_amd import _lib, ops
    lib = _lib.load()
    nbytes = -(-nbytes // 16384) * 16384
    ncopy = max(2, -(-ROTATE_BYTES // nbytes))
    bufs = [torch.randint(0, 255, (nbytes,), dtype=torch.uint8, device=dev) for _ in range(ncopy)]
    sink = torch.zeros(1, dtype=torch.int32, device=dev)
    out = {}
    for depth in (4, 8, 16):
        for wpc in (4, 8, 16):
            i = [0]

            def call():
                b = bufs[i[0]]
                i[0] = (i[0] + 1) % len(bufs)
                _lib.check(lib.dq_stream_read(ops._ptr(b), nbytes, wpc, depth, ops._ptr(sink), 0x9E3779B9,
                                              ops._stream()), "dq_stream_read")
            us = graph_time(call, ncopy, reps)
            out[f"{wpc}x{depth}KB"] = round(nbytes / us / 1e3, 1)
    del bufs
    return out, max(out.values())


def lds_probe_patterns():
    """Per-lane LDS byte offsets for dq_lds_read_probe (16-byte reads):
    - quads(i, j): lane quad i (lanes 4i..4i+3) reads bytes 0..63, quad j
      bytes 256..319 (the same 16 banks at another address), every other lane
      bytes 64..127 at its lane's slot (one address per slot: broadcasts on
      other banks). Only quads i and j can conflict, and they do exactly when
      one cycle serves both: every pair of the first half-wave's 8 quads, then
      quad 0 against each quad of the second half-wave;
    - contiguous: lane l at 16 l;
    - the prefill GEMM's Q4_K weight-fragment reads (64-byte rows, lane l on
      row l % 32, sub-plane l / 32 at a 16 KiB plane stride, item 0) with the
      earlier chunk swizzle ((row / 2) ^ (row / 8)) % 4 and the current
      (row / 4) % 4."""
    pats = []
    for i in range(8):
        for j in range(i + 1, 16):
            if j >= 8 and i > 0:
                continue
            offs = [64 + 16 * (l % 4) for l in range(64)]
            for l in range(4):
                offs[4 * i + l] = 16 * l
                offs[4 * j + l] = 256 + 16 * l
            pats.append((f"quads({i},{j})", offs))
    pats.append(("contiguous", [16 * l for l in range(64)]))
    for nm, swz in (("q4k_b_earlier_swizzle", lambda n: ((n >> 1) ^ (n >> 3)) & 3),
                    ("q4k_b_current_swizzle", lambda n: (n >> 2) & 3)):
        pats.append((nm, [16384 * (l >> 5) + 64 * (l & 31) + 16 * swz(l & 31) for l in range(64)]))
    return pats


# ------------------------------------------------------------------ CPU side

def host_description():
    """The host CPU as lscpu reports it (model, sockets, cores per socket,
    threads per core, total L3), and the threads this process may use."""
    import subprocess
    d = {}
    try:
        txt = subprocess.run(["lscpu"], capture_output=True, text=True, env=dict(os.environ, LC_ALL="C"),
                             timeout=20).stdout
        for line in txt.splitlines():
            k, _, v = line.partition(":")
            d[k.strip()] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    sockets = int(d.get("Socket(s)", "1") or 1)
    cps = int(d.get("Core(s) per socket", "0") or 0)
    tpc = int(d.get("Thread(s) per core", "1") or 1)
    # sysfs sums the distinct L3 instances; lscpu's "L3" line (newer
    # util-linux) is already that total
    l3_total = _sysfs_l3() or _parse_size(d.get("L3", ""))
    share = len(os.sched_getaffinity(0))
    if os.environ.get("OMP_NUM_THREADS", "").isdigit():
        share = min(share, int(os.environ["OMP_NUM_THREADS"]))
    phys = sockets * cps if cps else share
    return {"model": d.get("Model name", "?"), "sockets": sockets, "cores_per_socket": cps,
            "threads_per_core": tpc, "physical_cores": phys, "l3_bytes": l3_total,
            "cpu_share": share, "threads_used": max(1, min(phys, share))}


def _parse_size(txt):
    import re
    m = re.match(r"\s*([0-9.]+)\s*([KMG])i?B?", txt)
    if not m:
        return None
    return int(float(m.group(1)) * {"K": 1 << 10, "M": 1 << 20, "G": 1 << 30}[m.group(2)])


def _sysfs_l3():
    try:
        ids, total = set(), 0
        base = "/sys/devices/system/cpu"
        for c in os.listdir(base):
            p = os.path.join(base, c, "cache", "index3")
            if c.startswith("cpu") and os.path.isdir(p):
                sid = open(os.path.join(p, "shared_cpu_list")).read().strip()
                if sid not in ids:
                    ids.add(sid)
                    total += _parse_size(open(os.path.join(p, "size")).read().strip()) or 0
        return total or None
    except OSError:
        return None


def _best_of(fn, budget_s, min_calls=2):
    t_end = time.time() + budget_s
    best, calls = 1e30, 0
    while time.time() < t_end or calls < min_calls:
        t0 = time.perf_counter()
        fn()
        best = min(best, time.perf_counter() - t0)
        calls += 1
    return best, calls


def _dram_copies(w0, rot_bytes):
    """Distinct copies of a weight matrix totalling >= rot_bytes, so that
    calls rotating over them read DRAM, not the host's last-level cache
    (bench/kernel_bench.cpp:112-132)."""
    n = max(2, -(-rot_bytes // w0.nbytes))
    return [w0] + [np.roll(w0, k, axis=0) for k in range(1, n)]


def cpu_gemv(r, qtype, rows, cols, rot_bytes, budget_s, seed):
    from desireeia_amd import synth
    copies = _dram_copies(synth.gen_weights(qtype, rows, cols, seed), rot_bytes)
    x = synth.gen_act(cols, seed + 1)
    i = [0]

    def call():
        r.matmul(qtype, copies[i[0] % len(copies)], rows, cols, x)
        i[0] += 1
    best, calls = _best_of(call, budget_s)
    nbytes = rows * synth.row_bytes(qtype, cols)
    return nbytes / best / 1e9, best, calls, len(copies), len(copies) * copies[0].nbytes


def cpu_layer(r, budget_s=5.0):
    """Config 4's decode step on the CPU from the reference's own operators:
    matmul_q4_k / matmul_q6_k for the seven products (each quantizing its
    input per 256, as matvec does), kv_quantize_row for the new K/V rows,
    decode attention over 4097 positions from kv_dot_q8_0 / kv_axpy_q8_0 on
    the reference's thread pool, and RMSNorm / RoPE / SiLU / residuals in
    numpy (dense_forward.cpp:3897-4257 order). Four distinct layers (556 MB
    of weights) rotate so that weights come from DRAM."""
    from desireeia_amd import synth
    E, H, KV, HD, F, pos = 4096, 32, 8, 128, 14336, 4096
    shapes = {"q": (synth.Q4_K, H * HD, E), "k": (synth.Q4_K, KV * HD, E), "v": (synth.Q6_K, KV * HD, E),
              "o": (synth.Q4_K, E, H * HD), "gate": (synth.Q4_K, F, E), "up": (synth.Q4_K, F, E),
              "down": (synth.Q6_K, E, F)}
    base = {nm: synth.gen_weights(qt, rr, c, 40 + i) for i, (nm, (qt, rr, c)) in enumerate(shapes.items())}
    layers = [base] + [{nm: np.roll(w, k, axis=0) for nm, w in base.items()} for k in range(1, 4)]
    rng = np.random.default_rng(41)
    pb = KV * HD // 32 * 34
    kc = np.zeros((pos + 1) * pb, np.uint8)
    vc = np.zeros((pos + 1) * pb, np.uint8)
    kc[:pos * pb] = r.kv_quantize_row(rng.standard_normal(pos * KV * HD).astype(np.float32))
    vc[:pos * pb] = r.kv_quantize_row(rng.standard_normal(pos * KV * HD).astype(np.float32))
    an = (1 + 0.02 * rng.standard_normal(E)).astype(np.float32)
    fn = (1 + 0.02 * rng.standard_normal(E)).astype(np.float32)
    ts = np.float32(500000.0) ** np.float32(-2.0 / HD)
    th = np.float32(pos) * ts ** np.arange(HD // 2, dtype=np.float32)
    cs, sn = np.cos(th).astype(np.float32), np.sin(th).astype(np.float32)
    x0 = synth.gen_act(E, 42)
    state = {"i": 0}

    def norm(v, w):
        return v * (np.float32(1) / np.sqrt(np.float32(np.dot(v.astype(np.float64), v) / v.size) + np.float32(1e-5))) * w

    def rope(v, n):
        v = v.reshape(n, HD)
        a, b = v[:, :HD // 2].copy(), v[:, HD // 2:].copy()
        v[:, :HD // 2], v[:, HD // 2:] = a * cs - b * sn, a * sn + b * cs
        return v.reshape(-1)

    def step():
        w = layers[state["i"] % len(layers)]
        state["i"] += 1
        mm = lambda nm, v: r.matmul(shapes[nm][0], w[nm], shapes[nm][1], shapes[nm][2], v)
        xn = norm(x0, an)
        q, k, v = rope(mm("q", xn), H), rope(mm("k", xn), KV), mm("v", xn)
        kc[pos * pb:] = r.kv_quantize_row(k)
        vc[pos * pb:] = r.kv_quantize_row(v)
        ao = r.attn_decode(q, kc, vc, H, KV, HD, 0, pos)
        h = mm("o", ao) + x0
        xn2 = norm(h, fn)
        g, u = mm("gate", xn2), mm("up", xn2)
        with np.errstate(over="ignore"):
            act = (g / (np.float32(1) + np.exp(-g))) * u
        return mm("down", act) + h
    best, calls = _best_of(step, budget_s)
    return best, calls


def cpu_moe(r, budget_s=5.0):
    """Config 5 on the CPU as the reference's expert_ffn runs it
    (dense_forward.cpp:1524-1560, combine :4160-4181): per token, moe_route
    (top-2, renormalised) and, per selected expert, matmul_q4_k for up and
    gate, SiLU(gate) * up, matmul_q4_k for down, weighted sum. 64 tokens,
    8 experts of 14336 x 4096 Q4_K (792 MB of weights)."""
    from desireeia_amd import synth
    E, F, X, T = 4096, 14336, 8, 64
    wg = synth.gen_weights(synth.Q4_K, X * F, E, 50)
    wu = synth.gen_weights(synth.Q4_K, X * F, E, 51)
    wd = synth.gen_weights(synth.Q4_K, X * E, F, 52)
    x = synth.gen_act((T, E), 53)
    lg = synth.gen_act((T, X), 54)

    def call():
        out = np.zeros((T, E), np.float32)
        for t in range(T):
            ids, wts = r.moe_route(lg[t], 2, True)
            for e, wt in zip(ids, wts):
                e = int(e)
                u = r.matmul(synth.Q4_K, wu[e * F:(e + 1) * F], F, E, x[t])
                g = r.matmul(synth.Q4_K, wg[e * F:(e + 1) * F], F, E, x[t])
                with np.errstate(over="ignore"):
                    h = (g / (np.float32(1) + np.exp(-g))) * u
                out[t] += np.float32(wt) * r.matmul(synth.Q4_K, wd[e * E:(e + 1) * E], E, F, h)
        return out
    best, calls = _best_of(call, budget_s, min_calls=1)
    return best, calls


def cpu_baseline(budget_s=12.0):
    """The reference's own CPU operators (oracle/_ref, compiled from its
    sources) timed on this host: `value` is matmul_q4_k at the headline's up
    shape; `rows` cover the other configurations. Threads = the host's
    physical cores, capped at this process's CPU share; the GEMV rows rotate
    distinct weight copies totalling >= 4x the host's L3 (DRAM regime), best
    of repeated calls (bench/kernel_bench.cpp:40-53, 112-132)."""
    from desireeia_amd import synth
    from oracle import oracle as orc
    host = host_description()
    r = orc.ref()
    if r is None:
        # the compiled reference is absent: time the oracle's scalar port on a sample
        o = orc.oracle()
        rows, cols = 14336, 4096
        w = synth.gen_weights(synth.Q4_K, rows, cols, seed=99)
        x = synth.gen_act(cols, 100)
        best, calls = _best_of(lambda: o.matmul(synth.Q4_K, w, rows, cols, x, 0, 512), budget_s)
        nbytes = rows * synth.row_bytes(synth.Q4_K, cols)
        return {"value": round(nbytes / (best * rows / 512.0) / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
                "sample": f"Q4_K GEMV 14336x4096, rows 0..511 timed and scaled, best of {calls}", "host": host}
    threads = host["threads_used"]
    r.set_threads(threads)
    rot = max(4 * (host["l3_bytes"] or (64 << 20)), 264 << 20)
    gbs, best, calls, ncopy, wset = cpu_gemv(r, synth.Q4_K, 14336, 4096, rot, budget_s, 99)
    out = {"value": round(gbs, 3), "unit": "GB/s", "cores": threads, "kind": "reference",
           "sample": f"Q4_K GEMV 14336x4096 (matmul_q4_k incl. its per-256 activation quantization), "
                     f"{ncopy} distinct weight copies ({wset >> 20} MB, >= 4x L3), best of {calls} calls over "
                     f"{budget_s:.0f} s, {threads} threads",
           "host": host}
    rows = {}
    gbs, best, calls, ncopy, wset = cpu_gemv(r, synth.Q8_0, 4096, 4096, rot, 3.0, 31)
    rows["gemv_q80_4096x4096"] = {"GBps": round(gbs, 2), "us": round(best * 1e6, 1),
                                  "sample": f"matmul_q8_0 (config 1), {ncopy} copies ({wset >> 20} MB), best of {calls}"}
    log(f"cpu reference gemv_q80: {rows['gemv_q80_4096x4096']}")
    rows.update(cpu_rows(r))
    best, calls = cpu_layer(r)
    rows["layer_q4km_pos4096"] = {"ms_per_layer": round(best * 1e3, 3), "layers_per_s": round(1.0 / best, 1),
                                  "GBps": round((LAYER_WEIGHT_BYTES + KV_READ_BYTES) / best / 1e9, 1),
                                  "sample": f"config 4 decode step from the reference's matmul_q4_k/q6_k, "
                                            f"kv_quantize_row, kv_dot/kv_axpy attention; numpy glue; best of {calls}"}
    log(f"cpu reference layer: {rows['layer_q4km_pos4096']}")
    best, calls = cpu_moe(r)
    rows["moe_8x2_64tok"] = {"ms_per_call": round(best * 1e3, 1), "tokens_per_s": round(64 / best, 1),
                             "sample": f"config 5 as expert_ffn: moe_route + matmul_q4_k per token and expert, "
                                       f"best of {calls}"}
    log(f"cpu reference moe: {rows['moe_8x2_64tok']}")
    out["rows"] = rows
    return out


def cpu_rows(r, budget_s=3.0):
    """The reference's CPU path for the prefill GEMM (matmul_batch, Q4_K
    14336x4096, 512 tokens), prefill attention (attention_prefill_q8, 512
    tokens after 3584 cached positions, 32/8 heads of 128) and the output-head
    GEMV (matmul_q6_k 128256x4096). Best of repeated calls over budget_s each."""
    from desireeia_amd import synth
    from oracle import oracle as orc
    rows = {}
    R, C, T = 14336, 4096, 512
    w = synth.gen_weights(synth.Q4_K, R, C, seed=21)
    x = synth.gen_act((T, C), 22)
    best, calls = _best_of(lambda: r.matmul_batch(synth.Q4_K, w, R, C, x, T), budget_s)
    rows["gemm_q4k"] = {"TFLOPs": round(2.0 * T * R * C / best / 1e12, 4), "ms": round(best * 1e3, 2),
                        "sample": f"matmul_batch Q4_K {T}x{C} . {C}x{R}, best of {calls}"}
    del w, x
    hd, nkv, nh, pos0, T = 128, 8, 32, 3584, 512
    rng = np.random.default_rng(9)
    o = orc.oracle()
    kc = o.kv_quantize_row(rng.standard_normal((pos0 + T) * nkv * hd).astype(np.float32))
    vc = o.kv_quantize_row(rng.standard_normal((pos0 + T) * nkv * hd).astype(np.float32))
    q = rng.standard_normal((T, nh * hd)).astype(np.float32)
    best, calls = _best_of(lambda: r.attn_prefill(q, kc, vc, T, nh, nkv, hd, pos0), budget_s)
    keys = T * (pos0 + 1) + T * (T - 1) // 2
    rows["attn_prefill_512_after_3584"] = {"TFLOPs_alg": round(4.0 * hd * nh * keys / best / 1e12, 4),
                                           "ms": round(best * 1e3, 2),
                                           "sample": f"attention_prefill_q8, best of {calls}"}
    del kc, vc, q
    R, C = 128256, 4096
    w = synth.gen_weights(synth.Q6_K, R, C, seed=70)
    xv = synth.gen_act(C, 71)
    best, calls = _best_of(lambda: r.matmul(synth.Q6_K, w, R, C, xv), budget_s)
    rows["head_q6k_128256x4096"] = {"GBps": round(R * synth.row_bytes(synth.Q6_K, C) / best / 1e9, 2),
                                    "ms": round(best * 1e3, 2), "sample": f"matmul_q6_k, best of {calls}"}
    for k, v in rows.items():
        log(f"cpu reference {k}: {v}")
    return rows


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--only", default=None, help="profile helper: run one kernel N times (q4k_up, q4k_down, ...)")
    ap.add_argument("--no-cpu", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the kernels run on one GPU's share).",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from desireeia_amd import _lib, synth
    _lib.load()
    dev = torch.device("cuda:0")

    shapes = {
        "q4k_up": (synth.Q4_K, 14336, 4096), "q4k_down": (synth.Q4_K, 4096, 14336),
        "q40_up": (synth.Q4_0, 14336, 4096), "q40_down": (synth.Q4_0, 4096, 14336),
        "q80": (synth.Q8_0, 4096, 4096),
        "q6k_down": (synth.Q6_K, 4096, 14336),
    }
    if args.only == "copy":
        # plain device copy of a known size: the calibration kernel for the
        # FETCH_SIZE / WRITE_SIZE counters (33,030,144 bytes read and written)
        src = torch.empty(33030144, dtype=torch.uint8, device=dev).fill_(1)
        dst = torch.empty_like(src)
        for _ in range(args.steps):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy: {args.steps} x {src.numel()} bytes")
        return
    if args.only == "lds_phases":
        # one dispatch per pattern, to be run under a SQ_LDS_BANK_CONFLICT
        # counter pass (the dispatch order is logged)
        lib = _lib.load()
        from desireeia_amd import ops
        sink = torch.zeros(1, dtype=torch.int32, device=dev)
        for name, offs in lds_probe_patterns():
            d_off = torch.tensor(offs, dtype=torch.int32, device=dev)
            _lib.check(lib.dq_lds_read_probe(ops._ptr(d_off), 2000, 1024, 0, ops._ptr(sink), 0x9E3779B9,
                                             ops._stream()), "dq_lds_read_probe")
            torch.cuda.synchronize()
            log(f"lds pattern: {name}")
        return
    if args.only == "ceiling":
        for nb in (33103872, 17858560):
            per, best = stream_read_ceiling(dev, nb)
            log(f"stream read {nb} B: {per} GB/s by waves per CU; best {best} GB/s ({best / HBM_PEAK_GBS:.3f})")
        return
    gemm_shapes = {"gemm_q4k": (synth.Q4_K, 14336, 4096, 512), "gemm_q6k": (synth.Q6_K, 4096, 14336, 512),
                   "gemm_q80": (synth.Q8_0, 14336, 4096, 512)}
    if args.only in gemm_shapes or (args.only or "").replace("_tiles", "") in gemm_shapes:
        qt, r, c, t = gemm_shapes[args.only.replace("_tiles", "")]
        g = GemmCase(qt, r, c, t, 21, dev, tiles=args.only.endswith("_tiles"))
        us = graph_time(g.kernel, 10, max(1, args.steps // 10))
        us_step = graph_time(g.step, 10, max(1, args.steps // 10))
        log(f"{args.only}: gemm kernel {us:.1f} us = {g.flops() / us / 1e6:.1f} TFLOP/s; "
            f"quantize+gemm {us_step:.1f} us")
        return
    if args.only == "layer":
        lc = LayerCase(dev)
        us = graph_time(lc.step, 1, max(1, args.steps // len(lc.layers))) / len(lc.layers)
        log(f"layer: {us:.1f} us/layer, {lc.bytes_per_layer() / us / 1e3:.1f} GB/s")
        return
    if args.only == "moe":
        mc = MoeCase(dev)
        us = graph_time(mc.step, 4, max(1, args.steps // 4))
        log(f"moe: {us:.1f} us/call, {mc.bytes() / us / 1e3:.1f} GB/s, {mc.n_tok / us * 1e6:.0f} tok/s")
        return
    if args.only == "attn":
        ac = AttnCase(dev)
        us = graph_time(ac.kernel, len(ac.caches), max(1, args.steps // len(ac.caches)))
        log(f"attn: {us:.2f} us, {KV_READ_BYTES / us / 1e3:.1f} GB/s")
        return
    if args.only == "head":
        hc = HeadCase(dev)
        us = graph_time(hc.logits_step, 4, max(1, args.steps // 4))
        us_sel = graph_time(hc.select_step, 4, max(1, args.steps // 4))
        log(f"head: logits {us:.1f} us ({hc.bytes() / us / 1e3:.1f} GB/s), top-104 + draw {us_sel:.1f} us")
        return
    if args.only == "attn_prefill":
        pc = AttnPrefillCase(dev)
        us = graph_time(pc.kernel, 4, max(1, args.steps // 4))
        log(f"attn_prefill: {us:.1f} us, {pc.flops() / us / 1e6:.1f} TFLOP/s (algorithmic)")
        return
    if args.only in ("layer_prefill", "layer_prefill_tiles"):
        lp = LayerPrefillCase(dev, tiles=args.only.endswith("_tiles"))
        us = graph_time(lp.step, 1, max(1, args.steps))
        log(f"layer_prefill: {us:.1f} us/layer, {lp.n_tok / us * 1e6:.0f} tok/s, {lp.flops() / us / 1e6:.1f} TFLOP/s")
        return
    if args.only == "step":  # the headline step: fp32 activation, quantize + GEMV in one launch, up then down
        up = GemvCase(synth.Q4_K, 14336, 4096, 11, dev)
        down = GemvCase(synth.Q4_K, 4096, 14336, 12, dev)

        def fused():
            up.step()
            down.step()
        per = max(len(up.mats), len(down.mats))
        us = graph_time(fused, per, max(1, args.steps // per))
        log(f"step: {us:.2f} us, {(step_bytes(synth.Q4_K, 14336, 4096) + step_bytes(synth.Q4_K, 4096, 14336)) / us / 1e3:.1f} GB/s")
        return
    if args.only and args.only.endswith("_f32") and args.only[:-4] in shapes:
        qt, r, c = shapes[args.only[:-4]]
        case = GemvCase(qt, r, c, 11, dev)
        us, gbs = kernel_stats(case, launches=args.steps, fp32=True)
        log(f"{args.only}: {us:.2f} us/launch, {gbs:.1f} GB/s")
        return
    if args.only:
        qt, r, c = shapes[args.only]
        case = GemvCase(qt, r, c, 11, dev)
        us, gbs = kernel_stats(case, launches=args.steps)
        log(f"{args.only}: {us:.2f} us/launch, {gbs:.1f} GB/s")
        return

    cases = {k: GemvCase(qt, r, c, 11 + i, dev) for i, (k, (qt, r, c)) in enumerate(shapes.items())}

    # ---- headline: Q4_K decode FFN GEMVs (up 14336x4096 + down 4096x14336), quantize + GEMV each.
    # One graph holds exactly --steps steps (each on the next weight copy); it is
    # replayed REPLAYS times, each replay timed on its own, bracketed by
    # synchronisations; ms_per_step is the median replay.
    up, down = cases["q4k_up"], cases["q4k_down"]

    def step():
        up.step()
        down.step()

    REPLAYS = 10
    n_steps = max(1, args.steps)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    per_replay = replay_times(step, n_steps, REPLAYS, warmup_reps=1)
    wall = time.perf_counter() - t0
    srt = sorted(per_replay)
    us_med = 0.5 * (srt[(REPLAYS - 1) // 2] + srt[REPLAYS // 2])
    us_best = srt[0]
    ms_per_step = us_med / 1e3
    bytes_step = step_bytes(synth.Q4_K, 14336, 4096) + step_bytes(synth.Q4_K, 4096, 14336)
    value = bytes_step / (ms_per_step * 1e-3) / 1e9
    distinct = min(n_steps, len(up.mats)) * up.mats[0].buf.numel() + min(n_steps, len(down.mats)) * down.mats[0].buf.numel()
    log(f"headline step: median {us_med:.2f} us, best {us_best:.2f} us over {REPLAYS} replays of {n_steps} steps")

    # ---- per-kernel figures
    extra = {}
    for k, c in cases.items():
        us, gbs = kernel_stats(c)
        extra[k] = {"shape": f"{c.rows}x{c.cols}", "kernel_us": round(us, 3), "kernel_GBps": round(gbs, 1),
                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 4)}
        log(f"{k}: {us:.2f} us  {gbs:.1f} GB/s  ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    # the two launches of the headline step, each alone (fp32 activation, quantized in-kernel)
    for k in ("q4k_up", "q4k_down"):
        c = cases[k]
        us, gbs = kernel_stats(c, fp32=True)
        extra[k + "_f32"] = {"shape": f"{c.rows}x{c.cols}", "kernel_us": round(us, 3), "kernel_GBps": round(gbs, 1),
                             "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                             "bytes_per_launch": step_bytes(c.qtype, c.rows, c.cols)}
        log(f"{k} fp32 activation: {us:.2f} us  {gbs:.1f} GB/s  ({100 * gbs / HBM_PEAK_GBS:.1f}% of HBM peak)")
    # what a plain streaming read of the same size achieves on this device
    ceil = {}
    for nm, nb in (("33MB", bytes_step // 2), ("17.8MB", 17858560)):
        per, best = stream_read_ceiling(dev, nb)
        ceil[nm] = {"bytes": nb, "GBps_by_shape": per, "best_GBps": best,
                    "frac_hbm": round(best / HBM_PEAK_GBS, 4)}
        log(f"stream-read ceiling {nm}: {best} GB/s ({per})")
    extra["stream_read_ceiling"] = ceil
    # config 3: prefill GEMM, kernel alone and with the activation quantization
    for k, (qt, r, c, t) in gemm_shapes.items():
        g = GemmCase(qt, r, c, t, 21, dev)
        kt = replay_times(g.kernel, 10, 10)
        us = sorted(kt)[len(kt) // 2]
        us_q = sorted(replay_times(g.step, 10, 10))[5]
        tf = g.flops() / us / 1e6
        extra[k] = {"shape": f"{t}x{c} . {c}x{r}", "kernel_us": round(us, 2), "kernel_us_best": round(min(kt), 2),
                    "TFLOPs": round(tf, 1), "frac_fp16_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
                    "frac_int8_mfma": round(tf / INT8_PEAK_TOPS, 4),
                    "quantize_plus_gemm_us": round(us_q, 2),
                    "quantize_plus_gemm_TFLOPs": round(g.flops() / us_q / 1e6, 1)}
        log(f"{k}: {us:.1f} us  {tf:.1f} TFLOP/s; with the activation quantization {us_q:.1f} us")
        del g
        # the same product on the opt-in tile copy of the weights (dq_gemm_tiles_pack)
        g = GemmCase(qt, r, c, t, 21, dev, tiles=True)
        kt = replay_times(g.kernel, 10, 10)
        us = sorted(kt)[len(kt) // 2]
        us_q = sorted(replay_times(g.step, 10, 10))[5]
        tf = g.flops() / us / 1e6
        extra[k + "_tiles"] = {"shape": f"{t}x{c} . {c}x{r}", "kernel_us": round(us, 2),
                               "kernel_us_best": round(min(kt), 2), "TFLOPs": round(tf, 1),
                               "frac_fp16_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
                               "frac_int8_mfma": round(tf / INT8_PEAK_TOPS, 4),
                               "quantize_plus_gemm_us": round(us_q, 2),
                               "quantize_plus_gemm_TFLOPs": round(g.flops() / us_q / 1e6, 1)}
        log(f"{k} (tile copy of the weights): {us:.1f} us  {tf:.1f} TFLOP/s; with the activation quantization "
            f"{us_q:.1f} us")
        del g
    # config 4: decode attention alone and the whole decoder layer
    ac = AttnCase(dev)
    us = graph_time(ac.kernel, len(ac.caches), 10)
    extra["attn_decode_4097"] = {"kernel_us": round(us, 3), "GBps": round(KV_READ_BYTES / us / 1e3, 1),
                                 "frac_hbm": round(KV_READ_BYTES / us / 1e3 / HBM_PEAK_GBS, 4)}
    log(f"attention (32/8 heads, 4097 positions): {us:.2f} us")
    del ac
    lc = LayerCase(dev)
    us = graph_time(lc.step, 1, 20) / len(lc.layers)
    gbs = lc.bytes_per_layer() / us / 1e3
    extra["layer_q4km_pos4096"] = {"us_per_layer": round(us, 2), "GBps": round(gbs, 1),
                                   "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "layers_per_s": round(1e6 / us, 1),
                                   "bytes_per_layer": lc.bytes_per_layer()}
    log(f"decoder layer: {us:.1f} us/layer  {gbs:.1f} GB/s")
    del lc
    mc = MoeCase(dev)
    us = graph_time(mc.step, 4, 10)
    gbs = mc.bytes() / us / 1e3
    extra["moe_8x2_64tok"] = {"us_per_call": round(us, 2), "GBps": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                              "tokens_per_s": round(mc.n_tok / us * 1e6, 1), "bytes_per_call": mc.bytes()}
    log(f"MoE expert FFN (8 experts, top-2, 64 tokens): {us:.1f} us  {gbs:.1f} GB/s")
    del mc
    # prefill (the layer path over a prompt chunk): attention alone and the layer
    pc = AttnPrefillCase(dev)
    us = graph_time(pc.kernel, 4, 5)
    tf = pc.flops() / us / 1e6
    extra["attn_prefill_512_after_3584"] = {
        "kernel_us": round(us, 2), "TFLOPs_alg": round(tf, 1), "frac_fp16_mfma_alg": round(tf / FP16_PEAK_TFLOPS, 4),
        "frac_fp16_mfma_issued": round(3 * tf / FP16_PEAK_TFLOPS, 4)}
    log(f"prefill attention (512 tokens after 3584): {us:.1f} us  {tf:.1f} TFLOP/s algorithmic")
    del pc
    lp = LayerPrefillCase(dev)
    us = graph_time(lp.step, 1, 5)
    tf = lp.flops() / us / 1e6
    extra["layer_prefill_q4km_512tok"] = {"us_per_layer": round(us, 1), "tokens_per_s": round(lp.n_tok / us * 1e6, 1),
                                          "TFLOPs_alg": round(tf, 1), "frac_fp16_mfma": round(tf / FP16_PEAK_TFLOPS, 4)}
    log(f"decoder layer prefill (512 tokens): {us:.1f} us/layer  {lp.n_tok / us * 1e6:.0f} tok/s  {tf:.1f} TFLOP/s")
    del lp
    # the same layer with tile copies of its matrices for the products (dq_gemm_tiles_pack)
    lp = LayerPrefillCase(dev, tiles=True)
    us = graph_time(lp.step, 1, 5)
    tf = lp.flops() / us / 1e6
    extra["layer_prefill_q4km_512tok_tiles"] = {"us_per_layer": round(us, 1),
                                                "tokens_per_s": round(lp.n_tok / us * 1e6, 1),
                                                "TFLOPs_alg": round(tf, 1),
                                                "frac_fp16_mfma": round(tf / FP16_PEAK_TFLOPS, 4)}
    log(f"decoder layer prefill (512 tokens, tile copies of the weights): {us:.1f} us/layer  "
        f"{lp.n_tok / us * 1e6:.0f} tok/s  {tf:.1f} TFLOP/s")
    del lp
    hc = HeadCase(dev)
    us = graph_time(hc.logits_step, 4, 5)
    us_sel = graph_time(hc.select_step, 4, 5)
    gbs = hc.bytes() / us / 1e3
    extra["head_q6k_128256x4096"] = {"logits_us": round(us, 2), "GBps": round(gbs, 1),
                                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "topk104_draw_us": round(us_sel, 2)}
    log(f"output head 128256x4096 Q6_K: {us:.1f} us  {gbs:.1f} GB/s; top-104 + draw {us_sel:.1f} us")
    del hc
    # the dominant kernel of the timed step: the down launch (4096x14336, the
    # longer of the two), fp32 activation quantized in-kernel
    dom = extra["q4k_down_f32"]
    roofline = {"bound": "hbm", "achieved": dom["kernel_GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(dom["kernel_GBps"] / HBM_PEAK_GBS, 4), "traffic": recorded_traffic(),
                "traffic_source": os.path.relpath(TRAFFIC_FILE, ROOT),
                "kernel": "gemv_flat16_kernel (dq_gemv_f32, Q4_K 4096x14336: per-256 activation quantization "
                          "in-kernel + GEMV), the down launch of the headline step",
                "launch_us": dom["kernel_us"], "bytes_per_launch": dom["bytes_per_launch"],
                "ceiling_same_size_GBps": ceil["33MB"]["best_GBps"]}

    cpu = None if args.no_cpu else cpu_baseline()

    out = {
        "metric": METRIC, "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": n_steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int8", "data": "synthetic",
        "config": {"workload": "config 2: Q4_K decode GEMV, up 14336x4096 + down 4096x14336, "
                               "per-256 activation quantization + GEMV per matrix (one launch each)",
                   "bytes_per_step": bytes_step, "frac_hbm_step": round(value / HBM_PEAK_GBS, 4),
                   "replays": REPLAYS, "steps_per_replay": n_steps,
                   "us_per_step_median": round(us_med, 3), "us_per_step_best": round(us_best, 3),
                   "us_per_step_replays": [round(t, 3) for t in per_replay],
                   "distinct_weight_bytes": int(distinct), "wall_s": round(wall, 3)},
        "roofline": roofline, "cpu_baseline": cpu, "extra": extra,
    }
    print(json.dumps(out))


if __name__ == "__main__":
    main()
