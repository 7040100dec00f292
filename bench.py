"""Benchmark of the quantized-projection path on one MI355X.

Headline (`value`): GGUF Q4_K matvec, 4096 -> 14336, M = 1, in GB/s of algorithmic
bytes (raw weight blocks + activations read + outputs written) with the inputs
resident in HBM.  A step is one call of the hot path on one weight copy; the
copies rotate through a pool of more than 1 GiB, so no timed call is served from
the 256 MB Infinity Cache.

Method, for every workload: W warmup calls, then R = 10 repetitions of
L = max(--steps, 200) back-to-back calls, each repetition timed with HIP events
recorded on the stream the calls are issued on; the per-call time is the median
over the repetitions.  The same L calls are also captured once into a HIP graph
on that stream and the graph replayed R times ("graph" figures: the host's
issue cost is then out of the picture).  `value` and `ms_per_step` are the
stream figures.  One window of exactly --steps calls between two stream
synchronisations is reported beside them.

Also reported under "extra":
* the Q8_0 4096x4096 M=1 matvec, the fused SiLU(gate)*up + Q4_K 14336 -> 4096
  down projection, and Q4_K 20480 -> 4096 (k above 16384: the per-element path);
* the M = 16 block-verify products (Q4_K 4096 -> 14336 with bf16 and f32
  activations, Q8_0 4096 -> 4096 with f32 activations, raw blocks and 16-row
  tiles), the vocab-sized LM head at M = 1 and M = 16, and that head plus the
  argmax of every row;
* the 6-layer draft decoder's 16-token block forward over a 2048-position
  context (HIP graph replay and eager), in us per block, draft tokens/s and
  GB/s of algorithmic bytes (every weight, the context K/V, inputs and outputs
  once per block);
* the target side of the verify loop: one token through a 6-layer dense target
  of the draft's shape over a 2048-position K/V cache, with three captured
  states and the vocab-sized LM head (GB/s of every weight and the cache read
  once);
* ceilings: an empty kernel, and the fastest plain streaming read
  (lg_bench_read_shape) of 17.9, 33.1 and 350.7 MB buffers through the same kind
  of rotating pool, over a sweep of read shapes (threads per workgroup, loads in
  flight per thread, one-shot or persistent grid, plain or nontemporal loads);
  the headline's roofline carries its fraction of both 8 TB/s and the best read
  of its own byte count.

`cpu_baseline`: the oracle (the C restatement of the reference's CPU and shader
arithmetic) on the host cores: Q8_0 dequant_to_f32 of the 4096x4096 tensor, the
f32 matvec in proj.comp order on 4096x4096 f32 weights, the fused Q8_0 matvec in
proj_q8_0.comp order on 4096x4096, and the fused Q4_K matvec in proj_q4k.comp
order on the headline workload, each on one thread and on the process's CPU share.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-extra] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
import platform
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "laguna-raw-halo-strix_amd"))

import laguna_hip as lh  # noqa: E402
import synth  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "Q4_K/Q8_0 matvec HBM GB/s (% of peak) M=1; 6-layer draft block fwd µs"
POOL_BYTES = 1 << 30
REPS = 10
MIN_LAUNCHES = 200
CAPTURE_THREAD_LOCAL = 1


class Hip:
    """HIP events, stream capture and graphs through the runtime the library uses."""

    def __init__(self):
        h = ctypes.CDLL("libamdhip64.so")
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        h.hipEventCreate.argtypes = [pvp]
        h.hipEventRecord.argtypes = [vp, vp]
        h.hipEventSynchronize.argtypes = [vp]
        h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), vp, vp]
        h.hipEventDestroy.argtypes = [vp]
        h.hipStreamBeginCapture.argtypes = [vp, ctypes.c_int]
        h.hipStreamEndCapture.argtypes = [vp, pvp]
        h.hipGraphInstantiate.argtypes = [pvp, vp, vp, vp, ctypes.c_size_t]
        h.hipGraphLaunch.argtypes = [vp, vp]
        h.hipGraphExecDestroy.argtypes = [vp]
        h.hipGraphDestroy.argtypes = [vp]
        self.h = h
        self.a, self.b = self._event(), self._event()

    def _event(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def time_ms(self, stream, fn):
        """Elapsed GPU time of the work fn() issues on `stream`."""
        assert self.h.hipEventRecord(self.a, stream) == 0
        fn()
        assert self.h.hipEventRecord(self.b, stream) == 0
        assert self.h.hipEventSynchronize(self.b) == 0
        ms = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), self.a, self.b) == 0
        return ms.value

    def capture(self, stream, fn):
        """A graph executable holding the work fn() issues on `stream`."""
        g, ge = ctypes.c_void_p(), ctypes.c_void_p()
        assert self.h.hipStreamBeginCapture(stream, CAPTURE_THREAD_LOCAL) == 0
        try:
            fn()
        finally:
            st = self.h.hipStreamEndCapture(stream, ctypes.byref(g))
        assert st == 0, f"hipStreamEndCapture {st}"
        assert self.h.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0) == 0
        self.h.hipGraphDestroy(g)
        return ge


def _pool(ctx, raw, tiled=None):
    """Copies of `raw` (device buffers) filling more than POOL_BYTES; `tiled` =
    (dtype, k, n) repacks each copy into 16-row tiles."""
    copies = max(2, -(-POOL_BYTES // raw.nbytes))
    pool = []
    for _ in range(copies):
        b = lh.GpuBuffer(ctx, raw.nbytes)
        b.upload(raw)
        if tiled is not None:
            t = lh.repack_tiled(ctx, b, *tiled)
            ctx.sync()
            b.free()
            b = t
        pool.append(b)
    return pool, copies * raw.nbytes


_DRAFT = {}


def draft_model(seed, cfg):
    """The random-init draft (synth.dflash_model), generated once per process: the
    draft-block workloads and the target workload share its layers."""
    key = (seed, cfg.n_layers)
    if key not in _DRAFT:
        _DRAFT[key] = synth.dflash_model(seed, cfg, cfg.n_layers)
    return _DRAFT[key]


class Workload:
    name = ""
    bytes_per_call = 0
    graph_mode = True  # the calls can be captured into a HIP graph
    kernel = None      # the kernel a rocprof trace of this workload shows

    def setup(self, ctx):
        raise NotImplementedError

    def step(self, i, stream):
        raise NotImplementedError

    def teardown(self):
        for p in getattr(self, "pool", []):
            p.free()
        self.pool = []


class MatvecM1(Workload):
    def __init__(self, dtype, k, n, seed, fused=False, kernel=None):
        self.dtype, self.k, self.n, self.seed, self.fused, self.kernel = dtype, k, n, seed, fused, kernel
        self.bytes_per_call = synth.weight_bytes(dtype, k, n) + 4 * k * (2 if fused else 1) + 4 * n
        tag = {lh.Q4_K: "Q4_K", lh.Q8_0: "Q8_0"}[dtype]
        self.name = (f"fused SiLU(gate)*up + {tag} matvec {k}->{n} M=1" if fused else f"{tag} matvec {k}->{n} M=1")

    def setup(self, ctx):
        k, n = self.k, self.n
        raw = synth.q4k_weight(self.seed, k, n) if self.dtype == lh.Q4_K else synth.q8_0_weight(self.seed, k, n)
        self.pool, self.pool_bytes = _pool(ctx, raw)
        self.x = lh.upload_f32(ctx, synth.normal(self.seed + 1, k))
        self.up = lh.upload_f32(ctx, synth.normal(self.seed + 2, k)) if self.fused else None
        self.c = lh.GpuBuffer(ctx, 4 * n)

    def step(self, i, stream):
        w = self.pool[i % len(self.pool)]
        L = lh.lib()
        if self.fused:
            lh.check(L.lg_dispatch_silu_mul_proj_quant(self.x.ptr, self.up.ptr, w.ptr, self.c.ptr, self.k, self.n,
                                                       self.dtype, stream))
        else:
            lh.check(L.lg_dispatch_proj_quant(self.x.ptr, w.ptr, self.c.ptr, self.k, self.n, self.dtype, stream))

    def teardown(self):
        super().teardown()
        for b in (self.x, self.up, self.c):
            if b is not None:
                b.free()


class BatchM16(Workload):
    def __init__(self, dtype, k, n, x_dtype, seed, m=16, tiled=False, kernel=None):
        self.dtype, self.k, self.n, self.x_dtype, self.seed, self.m = dtype, k, n, x_dtype, seed, m
        self.tiled, self.kernel = tiled, kernel
        xb = 2 if x_dtype == lh.BF16 else 4
        self.bytes_per_call = synth.weight_bytes(dtype, k, n) + m * k * xb + 4 * m * n
        tag = {lh.Q4_K: "Q4_K", lh.Q8_0: "Q8_0"}[dtype]
        self.name = (f"{tag} block-verify {k}->{n} M={m} x={'bf16' if x_dtype == lh.BF16 else 'f32'}"
                     + (" (16-row tiles)" if tiled else ""))

    def setup(self, ctx):
        k, n, m = self.k, self.n, self.m
        raw = synth.q4k_weight(self.seed, k, n) if self.dtype == lh.Q4_K else synth.q8_0_weight(self.seed, k, n)
        self.pool, self.pool_bytes = _pool(ctx, raw, (self.dtype, k, n) if self.tiled else None)
        x = synth.normal(self.seed + 0x100, m * k)
        if self.x_dtype == lh.BF16:
            u = x.view(np.uint32).astype(np.uint64)
            x = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        self.x = lh.upload_bytes(ctx, x.view(np.uint8))
        self.c = lh.GpuBuffer(ctx, 4 * m * n)

    def step(self, i, stream):
        w = self.pool[i % len(self.pool)]
        wt = lh.TILED[self.dtype] if self.tiled else self.dtype
        lh.check(lh.lib().lg_dispatch_proj_quant_batch(self.x.ptr, self.x_dtype, w.ptr, self.c.ptr, self.k, self.n,
                                                       self.m, wt, stream))

    def teardown(self):
        super().teardown()
        self.x.free()
        self.c.free()


class VerifyBlock(BatchM16):
    """Target-side block verify: the vocab-sized LM head over m draft hidden states
    (src/target.rs:580-605), then the device argmax of each row of logits
    (src/lib.rs:456-464); the indices stay on the device."""

    def __init__(self, k, n, seed, m=16):
        super().__init__(lh.Q4_K, k, n, lh.F32, seed, m)
        self.bytes_per_call += 4 * m * n  # the argmax reads the logits back
        self.name = f"Q4_K LM head {k}->{n} M={m} + argmax per row"

    def setup(self, ctx):
        super().setup(ctx)
        self.idx = lh.GpuBuffer(ctx, 4 * self.m)

    def step(self, i, stream):
        super().step(i, stream)
        lh.check(lh.lib().lg_dispatch_argmax(self.c.ptr, self.n, self.m, self.n, self.idx.ptr, stream))

    def teardown(self):
        super().teardown()
        self.idx.free()


class DFlashBlock(Workload):
    """The 6-layer draft decoder's block forward: 16 tokens over a 2048-position f32
    K/V context, random-init weights (Q4_K except Q8_0 attn_output), either replayed
    as the captured HIP graph or launched eagerly.  One forward reads every weight
    once (917 MB > the 256 MB Infinity Cache), so one model copy needs no rotation."""

    graph_mode = False  # the forward is itself a graph (or its eager launches)

    def __init__(self, m=16, ctx_len=2048, seed=0x5EED000A, graph=False, tiled=True):
        self.m, self.ctx_len, self.seed, self.as_graph, self.tiled = m, ctx_len, seed, graph, tiled
        self.cfg = lh.DFlashConfig()
        self.name = (f"DFlash 6-layer block forward, {m} tokens over {ctx_len}-position f32 KV "
                     f"({'HIP graph' if graph else 'eager'}, "
                     f"{'16-row tiles' if tiled else 'raw GGUF blocks'})")

    def setup(self, ctx, stream=None):
        cfg, m = self.cfg, self.m
        W, layers = draft_model(self.seed, cfg)
        feat, tok, kc, vc = synth.dflash_inputs(self.seed + 1, cfg, cfg.n_layers, m, self.ctx_len)
        nbytes = lambda a: np.asarray(a).nbytes
        wbytes = sum(nbytes(W[n]) for n in ("enc_aux_norm", "fc", "enc_output_norm", "output_norm"))
        wbytes += sum(nbytes(L[n]) for L in layers for n in lh.DFLASH_NORMS + lh.DFLASH_PROJ)
        kvbytes = sum(nbytes(a) for a in kc + vc)
        self.bytes_per_call = wbytes + kvbytes + feat.nbytes + tok.nbytes + 4 * m * cfg.n_embd
        self.model = lh.DFlashModel(ctx, cfg, W, layers, tiled=self.tiled)
        self.model.set_context(kc, vc)
        del W, layers, kc, vc
        self.fb, self.tb = lh.upload_f32(ctx, feat), lh.upload_f32(ctx, tok)
        self.ob = lh.GpuBuffer(ctx, 4 * m * cfg.n_embd)
        self.pool_bytes = self.bytes_per_call
        if self.as_graph and stream is None:
            self.own_stream = stream = lh.Stream()
        self.g = self.model.capture(self.fb, self.tb, m, self.ob, stream) if self.as_graph else None

    def step(self, i, stream):
        if self.g is not None:
            lh.check(lh.lib().lg_dflash_graph_launch(self.g.ptr, stream))
        else:
            self.model.forward_block_device(self.fb, self.tb, self.m, self.ob, stream=stream)

    def teardown(self):
        if self.g is not None:
            self.g.destroy()
        self.model.free()
        for b in (self.fb, self.tb, self.ob):
            b.free()


class Empty(Workload):
    def __init__(self, workgroups=256):
        self.wg = workgroups
        self.name = f"empty kernel, {workgroups} workgroups"
        self.kernel = "k_empty"

    def setup(self, ctx):
        self.pool, self.pool_bytes = [], 0

    def step(self, i, stream):
        lh.check(lh.lib().lg_bench_empty(self.wg, stream))


class Read(Workload):
    """A plain streaming read of `nbytes` through a rotating pool; `shape` =
    (threads per workgroup, 16-byte loads per thread per chunk, workgroups per CU of
    a persistent grid or 0 for one-shot, nontemporal loads), as lg_bench_read_shape."""

    def __init__(self, nbytes, shape=(256, 8, 0, 0)):
        self.bytes_per_call, self.shape = nbytes, tuple(shape)
        t, l, pc, nt = self.shape
        grid = f"persistent {pc}/CU" if pc else "one-shot"
        self.name = (f"streaming read of {nbytes / 1e6:.1f} MB ({t} threads x {l} loads = {t * l * 16 // 1024} KiB "
                     f"per chunk, {grid}{', nontemporal' if nt else ''})")
        self.kernel = "k_read"

    def setup(self, ctx):
        copies = max(2, -(-POOL_BYTES // self.bytes_per_call))
        self.pool = [lh.GpuBuffer(ctx, self.bytes_per_call) for _ in range(copies)]
        for p in self.pool:
            p.fill(1)
        ctx.sync()
        self.pool_bytes = copies * self.bytes_per_call

    def step(self, i, stream):
        w = self.pool[i % len(self.pool)]
        lh.check(lh.lib().lg_bench_read_shape(w.ptr, self.bytes_per_call, *self.shape, stream))


READ_SHAPES = [(t, l, pc, nt) for t in (256, 512, 1024) for l in (2, 4, 8, 16) for pc in (0, 1, 2)
               for nt in (0, 1) if not (pc and t * l > 8192)]
READ_SIZES = {"17.8MB": 17858560, "33.1MB": 33103872, "350MB": 350684672}


def ceiling_sweep(ctx, hip, reps=5, launches=MIN_LAUNCHES):
    """The fastest plain read of each byte count over READ_SHAPES: per size, one
    rotating pool, every shape timed as the workloads are (median of `reps` x
    `launches` back-to-back calls, HIP events on the stream)."""
    out = {}
    for tag, nbytes in READ_SIZES.items():
        wl = Read(nbytes)
        wl.setup(ctx)
        stream = lh.Stream()
        s = stream.ptr
        res = []
        for shape in READ_SHAPES:
            wl.shape = shape
            for i in range(3):
                wl.step(i, s)
            stream.sync()
            t = [1000.0 * hip.time_ms(s, lambda: [wl.step(r * launches + i, s) for i in range(launches)]) / launches
                 for r in range(reps)]
            res.append((statistics.median(t), shape))
        wl.teardown()
        stream.destroy()
        res.sort()
        us, best = res[0]
        base = next(u for u, sh in res if sh == (256, 8, 0, 0))
        out[tag] = {"bytes": nbytes, "best_us": round(us, 3), "best_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
                    "best_shape": {"threads": best[0], "loads": best[1], "per_cu": best[2], "nontemporal": best[3]},
                    "default_shape_us": round(base, 3), "shapes_tried": len(res),
                    "top5": [[round(u, 3), list(sh)] for u, sh in res[:5]]}
        print(f"# ceiling sweep {tag}: best {us:.3f} us {best} (default shape {base:.3f} us)", file=sys.stderr,
              flush=True)
    return out


class TargetToken(Workload):
    """Target-side verify step: one token through a dense target with the device K/V
    cache holding `ctx_len` positions (src/target.rs:298-578), the hidden states
    captured after layers 1, 3 and 5 (the draft's three features), then the Q4_K LM
    head over the vocabulary (src/target.rs:580-605).  Six layers of the draft's shape
    (hidden 4096, 32 Q / 8 KV heads of 128, FFN 14336, an attention gate), weights of
    trained magnitude: zero-mean Q4_K blocks (synth.centered_q4k, standard deviation
    0.02) with a ggml-quantized N(0, 0.02) Q8_0 attn_output, so the residual stream
    stays finite as in a real model; the six layers hold device copies of one set of
    values.  The cache holds N(0, 1) keys and values.  Every
    call appends position ctx_len (the cache length is reset before each), so each
    reads all weights once (1.2 GB, past the Infinity Cache)."""

    graph_mode = False  # the cache length is host state the call advances

    def __init__(self, ctx_len=2048, n_vocab=151936, seed=0x5EED000A):
        self.ctx_len, self.n_vocab, self.seed = ctx_len, n_vocab, seed
        self.name = f"dense target forward, 1 token over a {ctx_len}-position K/V cache, 6 layers + LM head {n_vocab}"
        self.kernel = None

    def setup(self, ctx):
        dc = lh.DFlashConfig()
        cfg = lh.TargetConfig(n_embd=dc.n_embd, n_heads=dc.n_heads, n_kv=dc.n_kv, head_dim=dc.head_dim,
                              n_ff=dc.n_ff, n_layers=dc.n_layers, n_vocab=self.n_vocab, rope_dim=dc.rope_dim)
        E, HD, KVD, FF, H = cfg.n_embd, cfg.head_dim, cfg.n_kv * cfg.head_dim, cfg.n_ff, cfg.n_heads
        shapes = {"attn_q": (E, H * HD), "attn_k": (E, KVD), "attn_v": (E, KVD), "attn_gate": (E, H),
                  "attn_output": (H * HD, E), "ffn_gate": (E, FF), "ffn_up": (E, FF), "ffn_down": (FF, E)}
        seeds = iter(synth.splitmix64(self.seed, 12))
        L = {n: np.ones(HD if n in ("attn_q_norm", "attn_k_norm") else E, np.float32) for n in lh.TARGET_NORMS}
        for p, (k, n) in shapes.items():
            sd = int(next(seeds))
            if p == "attn_output":
                L[p], L[p + "_dtype"] = synth.q8_0_weight(sd, k, n), lh.Q8_0
            else:
                L[p], L[p + "_dtype"] = synth.centered_q4k(sd, k * n // 256), lh.Q4_K
        # every layer uploads its own device copy of the same host arrays: the calls
        # read 6 distinct sets of weights (generating one set keeps the set-up short)
        layers = [dict(L) for _ in range(cfg.n_layers)]
        out = synth.centered_q4k(int(next(seeds)), cfg.n_embd * cfg.n_vocab // 256)
        onorm = np.ones(cfg.n_embd, np.float32)
        nbytes = lambda a: np.asarray(a).nbytes
        wbytes = sum(nbytes(L[n]) for L in layers for n in lh.TARGET_NORMS + lh.TARGET_PROJ) + out.nbytes
        kvd = cfg.n_kv * cfg.head_dim
        kvbytes = 2 * cfg.n_layers * (self.ctx_len + 1) * kvd * 4
        self.bytes_per_call = wbytes + kvbytes + onorm.nbytes + 4 * (cfg.n_embd * 5 + cfg.n_vocab)
        self.model = lh.TargetModel(ctx, cfg, layers, output_norm=onorm, output=out, output_dtype=lh.Q4_K)
        del layers, out
        self.cache = lh.TargetKvCache(self.model, self.ctx_len + 1)
        n = cfg.n_layers * (self.ctx_len + 1) * kvd
        self.cache.k.upload(synth.normal(self.seed + 8, n))
        self.cache.v.upload(synth.normal(self.seed + 9, n))
        self.x = lh.upload_f32(ctx, synth.normal(self.seed + 10, cfg.n_embd))
        self.capture = [1, 3, 5]
        self.cb = lh.GpuBuffer(ctx, 4 * len(self.capture) * cfg.n_embd)
        self.lb = lh.GpuBuffer(ctx, 4 * cfg.n_vocab)
        self.pool_bytes = self.bytes_per_call

    def step(self, i, stream):
        self.cache._c.len = self.ctx_len
        self.model.forward_token_device(self.x, self.capture, self.cb, self.lb, cache=self.cache, stream=stream)

    def teardown(self):
        self.model.free()
        self.cache.free()
        for b in (self.x, self.cb, self.lb):
            b.free()


HEAD_KERNEL = "k_q4k_m1_dig"
WORKLOADS = {
    "q4k_m1": lambda: MatvecM1(lh.Q4_K, 4096, 14336, 0x5EED0003, kernel=HEAD_KERNEL),
    "q8_0_m1": lambda: MatvecM1(lh.Q8_0, 4096, 4096, 0x5EED0001, kernel="k_q80_m1_dig"),
    "q4k_m1_4096": lambda: MatvecM1(lh.Q4_K, 4096, 4096, 0x5EED000F, kernel=HEAD_KERNEL),
    "q4k_down_silu": lambda: MatvecM1(lh.Q4_K, 14336, 4096, 0x5EED0005, fused=True, kernel="k_q4k_m1_wide"),
    "q4k_m1_k14336": lambda: MatvecM1(lh.Q4_K, 14336, 4096, 0x5EED0005, kernel="k_q4k_m1_wide"),
    "q4k_m1_k20480": lambda: MatvecM1(lh.Q4_K, 20480, 4096, 0x5EED000C, kernel="k_q4k_m1"),
    "q4k_m16_bf16": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.BF16, 0x5EED0008, kernel="k_q4k_mm"),
    "q4k_m16_f32": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.F32, 0x5EED0008, kernel="k_q4k_mm"),
    "q4k_m16_f32_tiled": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.F32, 0x5EED0008, tiled=True, kernel="k_q4k_mm"),
    "q8_0_m16_f32": lambda: BatchM16(lh.Q8_0, 4096, 4096, lh.F32, 0x5EED0009, kernel="k_q80_mm"),
    "q8_0_m16_f32_tiled": lambda: BatchM16(lh.Q8_0, 4096, 4096, lh.F32, 0x5EED0009, tiled=True, kernel="k_q80_mm"),
    # vocab-sized output projection (the LM head, src/target.rs:580-605): M=1 for one
    # token, M=16 to verify a 16-token draft block
    "q4k_lm_head_m1": lambda: MatvecM1(lh.Q4_K, 4096, 151936, 0x5EED000B, kernel=HEAD_KERNEL),
    "q4k_lm_head_m16": lambda: BatchM16(lh.Q4_K, 4096, 151936, lh.F32, 0x5EED000B, kernel="k_q4k_mm"),
    "lm_head_verify_m16": lambda: VerifyBlock(4096, 151936, 0x5EED000B),
    "dflash_block": lambda: DFlashBlock(graph=False),
    "dflash_block_graph": lambda: DFlashBlock(graph=True),
    # the same forward over the raw GGUF blocks as uploaded (no repack at load)
    "dflash_block_raw": lambda: DFlashBlock(graph=False, tiled=False),
    "target_token": lambda: TargetToken(),
    "ceil_empty": lambda: Empty(256),
    "ceil_read_17.8MB": lambda: Read(17858560),
    "ceil_read_33.1MB": lambda: Read(33103872),
    "ceil_read_350MB": lambda: Read(350684672),
}
EXTRA = ["q8_0_m1", "q4k_m1_4096", "q4k_down_silu", "q4k_m1_k14336", "q4k_m1_k20480", "q4k_m16_bf16", "q4k_m16_f32", "q4k_m16_f32_tiled",
         "q8_0_m16_f32", "q8_0_m16_f32_tiled", "q4k_lm_head_m1", "q4k_lm_head_m16", "lm_head_verify_m16",
         "dflash_block", "dflash_block_graph", "dflash_block_raw", "target_token", "ceil_empty"]


def time_workload(ctx, hip, wl, steps, warmup, launches=None):
    """Per-call us: median over REPS repetitions of `launches` back-to-back calls,
    issued from the host (stream) and replayed from one captured graph (graph), plus
    one window of exactly `steps` calls."""
    L = launches or max(steps, MIN_LAUNCHES)
    stream = lh.Stream()
    s = stream.ptr
    t0 = time.perf_counter()
    if isinstance(wl, DFlashBlock):
        wl.setup(ctx, stream)
    else:
        wl.setup(ctx)
    for i in range(warmup):
        wl.step(i, s)
    stream.sync()
    t_issue0 = time.perf_counter()
    ms_window = hip.time_ms(s, lambda: [wl.step(warmup + i, s) for i in range(steps)])
    reps = []
    for r in range(REPS):
        reps.append(1000.0 * hip.time_ms(s, lambda: [wl.step(r * L + i, s) for i in range(L)]) / L)
    host_s = time.perf_counter() - t_issue0
    us = statistics.median(reps)
    r = {"workload": wl.name, "us_per_call": round(us, 3), "launches_per_rep": L, "reps": REPS,
         "us_spread": [round(min(reps), 3), round(max(reps), 3)],
         "us_per_call_steps_window": round(1000.0 * ms_window / max(steps, 1), 3), "steps_window": steps}
    if wl.graph_mode:
        ge = hip.capture(s, lambda: [wl.step(i, s) for i in range(L)])
        hip.h.hipGraphLaunch(ge, s)
        stream.sync()
        g = [1000.0 * hip.time_ms(s, lambda: hip.h.hipGraphLaunch(ge, s)) / L for _ in range(REPS)]
        hip.h.hipGraphExecDestroy(ge)
        r["us_per_call_graph"] = round(statistics.median(g), 3)
    if wl.bytes_per_call:
        gbs = wl.bytes_per_call / (us * 1e-6) / 1e9
        r.update({"GBps": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
                  "bytes_per_call": wl.bytes_per_call, "pool_MB": round(wl.pool_bytes / 2 ** 20, 1)})
        if "us_per_call_graph" in r:
            r["GBps_graph"] = round(wl.bytes_per_call / (r["us_per_call_graph"] * 1e-6) / 1e9, 1)
    if isinstance(wl, DFlashBlock):
        r["draft_tokens_per_s"] = round(wl.m / (us * 1e-6), 1)
    if wl.kernel:
        r["kernel"] = wl.kernel
    r["host_wall_s"] = round(time.perf_counter() - t0, 3)
    r["host_issue_s"] = round(host_s, 3)
    wl.teardown()
    stream.sync()
    stream.destroy()
    return r


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


def cpu_threads():
    """The process's CPU share: OMP_NUM_THREADS when set, else the CPUs it may run on."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def _rate(fn, nbytes, budget_s):
    """Bytes per second of fn() repeated for at least budget_s (at least twice)."""
    reps, t = 0, 0.0
    while t < budget_s or reps < 2:
        t0 = time.perf_counter()
        fn()
        t += time.perf_counter() - t0
        reps += 1
    return reps * nbytes / t, reps, t


def cpu_baseline(budget_s=2.0):
    """The oracle on the host: three legs, each on one thread and on the CPU share."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    nthr = cpu_threads()
    legs = {}
    # 1. dequant_to_f32 of a Q8_0 tensor (src/dflash.rs:379-397), the load-time cost
    q8 = synth.q8_0_weight(0x5EED0001, 4096, 4096)
    n_el = 4096 * 4096
    for t in (1, nthr):
        fn = (lambda: orc.dequant_to_f32(q8, orc.Q8_0, n_el)) if t == 1 else (lambda: orc.dequant_q8_0_mt(q8, n_el, t))
        bps, reps, secs = _rate(fn, q8.nbytes, budget_s)
        legs[f"dequant_q8_0_4096x4096_t{t}"] = {"GBps": round(bps / 1e9, 4), "Melem_per_s": round(bps / q8.nbytes *
                                                                                                 n_el / 1e6, 1),
                                                "threads": t, "calls": reps, "seconds": round(secs, 2)}
    # 2. the f32 matvec in kernels/proj.comp order (the reference draft's projections)
    wf = synth.normal(0x5EED0101, 4096 * 4096, 0.02)
    xf = synth.normal(0x5EED0102, 4096)
    for t in (1, nthr):
        bps, reps, secs = _rate(lambda: orc.proj_f32(xf, wf, 4096, 4096, threads=t), wf.nbytes + 4 * 4096 + 4 * 4096,
                                budget_s)
        legs[f"proj_f32_4096x4096_t{t}"] = {"GBps": round(bps / 1e9, 4), "threads": t, "calls": reps,
                                            "seconds": round(secs, 2)}
    del wf
    # 3a. the fused Q8_0 matvec in kernels/proj_q8_0.comp order (4096 x 4096)
    x8 = synth.normal(0x5EED0002, 4096)
    for t in (1, nthr):
        bps, reps, secs = _rate(lambda: orc.proj_q8_0(x8, q8, 4096, 4096, threads=t), q8.nbytes + 4 * 4096 + 4 * 4096,
                                budget_s)
        legs[f"proj_q8_0_4096x4096_t{t}"] = {"GBps": round(bps / 1e9, 4), "threads": t, "calls": reps,
                                             "seconds": round(secs, 2)}
    # 3b. the fused Q4_K matvec in kernels/proj_q4k.comp order on the headline workload
    k, n = 4096, 14336
    q4 = synth.q4k_weight(0x5EED0003, k, n)
    x = synth.normal(0x5EED0004, k)
    nbytes = q4.nbytes + 4 * k + 4 * n
    for t in (1, nthr):
        bps, reps, secs = _rate(lambda: orc.proj_q4k(x, q4, k, n, threads=t), nbytes, budget_s)
        legs[f"proj_q4k_4096x14336_t{t}"] = {"GBps": round(bps / 1e9, 4), "threads": t, "calls": reps,
                                             "seconds": round(secs, 2)}
    head = legs[f"proj_q4k_4096x14336_t{nthr}"]
    return {"value": head["GBps"], "unit": "GB/s", "cores": nthr, "kind": "port",
            "cpu_model": cpu_model(), "cpu_count": os.cpu_count(), "legs": legs,
            "sample": f"oracle (C, -O2, no FMA contraction) on the host: Q8_0 dequant_to_f32 of 4096x4096, f32 "
                      f"proj.comp-order matvec 4096x4096, fused Q8_0 proj_q8_0.comp-order matvec 4096x4096, fused "
                      f"Q4_K proj_q4k.comp-order matvec 4096->14336 (the value); whole calls repeated for about "
                      f"{budget_s:.0f} s each on 1 and {nthr} threads"}


CAL_BYTES = 64 << 20  # lg_buf_copy size that hardware traffic counters are calibrated against


def traffic_from_profile(workload):
    """HBM bytes per launch of the workload's kernel, from the committed summary of
    two rocprofv3 --pmc runs of `bench.py --pmc` (FETCH_SIZE, then WRITE_SIZE, each
    scaled by what the counter reads for lg_buf_copy of CAL_BYTES); None if absent."""
    path = os.path.join(ROOT, "profiles", f"traffic_{workload}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            return int(float(line.split(":", 1)[1]))
    return None


def pmc_run(ctx, wl, steps):
    """For counter collection: three lg_buf_copy calls of CAL_BYTES (the calibration
    kernel) followed by `steps` calls of the workload, each on its own weight copy."""
    a, b = lh.GpuBuffer(ctx, CAL_BYTES), lh.GpuBuffer(ctx, CAL_BYTES)
    for _ in range(3):
        b.copy_from(a, CAL_BYTES)
    ctx.sync()
    a.free()
    b.free()
    wl.setup(ctx) if not isinstance(wl, DFlashBlock) else wl.setup(ctx, None)
    for i in range(steps):
        wl.step(i, None)
    ctx.sync()
    wl.teardown()
    print(json.dumps({"pmc_run": wl.name, "steps": steps, "calibration_copy_bytes": CAL_BYTES}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="q4k_m1", choices=sorted(WORKLOADS))
    ap.add_argument("--no-extra", action="store_true", help="time only the headline workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc", action="store_true",
                    help="counter-collection mode: calibration copies, then --steps calls of --workload")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(the projection path would shard by output rows; see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    ctx = lh.VulkanContext(0)
    if args.pmc:
        pmc_run(ctx, WORKLOADS[args.workload](), args.steps)
        return
    hip = Hip()
    wl = WORKLOADS[args.workload]()
    head = time_workload(ctx, hip, wl, args.steps, args.warmup)
    print(f"# {args.workload}: {head['us_per_call']} us/call (graph {head.get('us_per_call_graph')})",
          file=sys.stderr, flush=True)
    extra = {}
    if not args.no_extra:
        for name in EXTRA:
            if name != args.workload:
                w = WORKLOADS[name]()
                extra[name] = time_workload(ctx, hip, w, args.steps, max(3, args.warmup // 4))
                print(f"# {name}: {extra[name]['us_per_call']} us/call", file=sys.stderr, flush=True)
    if "GBps" in head:
        roof = {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": head["frac_of_peak"], "traffic": traffic_from_profile(args.workload),
                "us_per_call": head["us_per_call"], "algorithmic_bytes": head["bytes_per_call"],
                "kernel": wl.kernel}
    else:  # a workload that moves no data (the empty kernel)
        roof = {"bound": "launch", "us_per_call": head["us_per_call"], "kernel": wl.kernel}
    sweep = None if args.no_extra else ceiling_sweep(ctx, hip)
    ceil = sweep.get("33.1MB") if sweep and args.workload == "q4k_m1" else None
    if ceil:
        roof.update({"ceiling_read_GBps": ceil["best_GBps"], "frac_of_ceiling_read": round(head["GBps"] /
                                                                                              ceil["best_GBps"], 4),
                     "ceiling_read_us": ceil["best_us"], "ceiling_read_shape": ceil["best_shape"]})
    if "ceil_empty" in extra:
        roof["empty_launch_us"] = extra["ceil_empty"]["us_per_call"]
        roof["empty_launch_us_graph"] = extra["ceil_empty"].get("us_per_call_graph")
    line = {
        "metric": METRIC,
        "value": head.get("GBps"),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1000.0, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded SplitMix64: random valid Q4_K blocks, ggml-quantized Q8_0, N(0,1) activations)",
        "config": {"workload": head["workload"], "k": getattr(wl, "k", None), "n": getattr(wl, "n", None),
                   "m": getattr(wl, "m", 1),
                   "weight_pool_MB": head.get("pool_MB"), "parallelism": "single GPU",
                   "timing": f"median of {REPS} x {head['launches_per_rep']} back-to-back calls"},
        "graph_us_per_call": head.get("us_per_call_graph"),
        "roofline": roof,
        "extra": extra,
        "ceiling_sweep": sweep,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
