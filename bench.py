"""Benchmark of the quantized-projection path on one MI355X.

Headline (`value`): GGUF Q4_K matvec, 4096 -> 14336, M = 1, in GB/s of algorithmic
bytes (raw weight blocks + activations read + outputs written) with the inputs
resident in HBM.  A step is one call of the hot path on one weight copy; the
copies rotate through a pool of more than 1 GiB so that no timed call is served
from the 256 MB Infinity Cache.  Kernel time is taken with HIP events recorded on
the stream the kernels run on.

Also reported under "extra": the Q8_0 4096x4096 M=1 matvec, the fused
SiLU(gate)*up + Q4_K 14336 -> 4096 down projection, the M = 16 block-verify
products (Q4_K 4096 -> 14336 with bf16 and f32 activations, Q8_0 4096 -> 4096
with f32 activations), and the 6-layer draft decoder's 16-token block forward
over a 2048-position context (HIP graph replay and eager), in us per block, draft
tokens/s and GB/s of algorithmic bytes (every weight, the context K/V, inputs
and outputs once per block).

`cpu_baseline`: the same Q4_K matvec computed by the oracle (a C restatement of
kernels/proj_q4k.comp's per-element decode and f32 accumulation) on the host
cores, over a bounded sample of output rows.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload NAME] [--no-cpu]
"""
import argparse
import ctypes
import json
import os
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


class HipEvents:
    """hipEvent timing through the HIP runtime the library itself uses."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def new(self):
        e = ctypes.c_void_p()
        assert self.hip.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e, stream):
        assert self.hip.hipEventRecord(e, stream) == 0

    def elapsed_ms(self, a, b):
        assert self.hip.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


class Workload:
    name = ""
    bytes_per_call = 0

    def setup(self, ctx):
        raise NotImplementedError

    def step(self, ctx, i):
        raise NotImplementedError


class MatvecM1(Workload):
    def __init__(self, dtype, k, n, seed, fused=False):
        self.dtype, self.k, self.n, self.seed, self.fused = dtype, k, n, seed, fused
        wbytes = synth.weight_bytes(dtype, k, n)
        xbytes = 4 * k * (2 if fused else 1)
        self.bytes_per_call = wbytes + xbytes + 4 * n
        tag = {lh.Q4_K: "Q4_K", lh.Q8_0: "Q8_0"}[dtype]
        self.name = (f"fused SiLU(gate)*up + {tag} matvec {k}->{n} M=1" if fused else f"{tag} matvec {k}->{n} M=1")

    def setup(self, ctx):
        k, n = self.k, self.n
        raw = synth.q4k_weight(self.seed, k, n) if self.dtype == lh.Q4_K else synth.q8_0_weight(self.seed, k, n)
        copies = max(2, -(-POOL_BYTES // raw.nbytes))
        self.pool = []
        for _ in range(copies):
            b = lh.GpuBuffer(ctx, raw.nbytes)
            b.upload(raw)
            self.pool.append(b)
        self.pool_bytes = copies * raw.nbytes
        self.x = lh.upload_f32(ctx, synth.normal(self.seed + 1, k))
        self.up = lh.upload_f32(ctx, synth.normal(self.seed + 2, k)) if self.fused else None
        self.c = lh.GpuBuffer(ctx, 4 * n)

    def step(self, ctx, i):
        w = self.pool[i % len(self.pool)]
        if self.fused:
            lh.dispatch_silu_mul_proj_quant(ctx, self.x, self.up, w, self.c, self.k, self.n, self.dtype)
        else:
            lh.dispatch_proj_quant(ctx, self.x, w, self.c, self.k, self.n, self.dtype)


class BatchM16(Workload):
    def __init__(self, dtype, k, n, x_dtype, seed, m=16, tiled=False):
        self.dtype, self.k, self.n, self.x_dtype, self.seed, self.m = dtype, k, n, x_dtype, seed, m
        self.tiled = tiled
        xb = 2 if x_dtype == lh.BF16 else 4
        self.bytes_per_call = synth.weight_bytes(dtype, k, n) + m * k * xb + 4 * m * n
        tag = {lh.Q4_K: "Q4_K", lh.Q8_0: "Q8_0"}[dtype]
        self.name = (f"{tag} block-verify {k}->{n} M={m} x={'bf16' if x_dtype == lh.BF16 else 'f32'}"
                     + (" (16-row tiles)" if tiled else ""))

    def setup(self, ctx):
        k, n, m = self.k, self.n, self.m
        raw = synth.q4k_weight(self.seed, k, n) if self.dtype == lh.Q4_K else synth.q8_0_weight(self.seed, k, n)
        copies = max(2, -(-POOL_BYTES // raw.nbytes))
        self.pool = []
        for _ in range(copies):
            b = lh.GpuBuffer(ctx, raw.nbytes)
            b.upload(raw)
            if self.tiled:  # the same bytes, permuted into 16-row tiles
                t = lh.repack_tiled(ctx, b, self.dtype, k, self.n)
                ctx.sync()
                b.free()
                b = t
            self.pool.append(b)
        self.pool_bytes = copies * raw.nbytes
        x = synth.normal(self.seed + 0x100, m * k)
        if self.x_dtype == lh.BF16:
            u = x.view(np.uint32).astype(np.uint64)
            x = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        self.x = lh.upload_bytes(ctx, x.view(np.uint8))
        self.c = lh.GpuBuffer(ctx, 4 * m * n)

    def step(self, ctx, i):
        w = self.pool[i % len(self.pool)]
        lh.dispatch_proj_quant_batch(ctx, self.x, self.x_dtype, w, self.c, self.k, self.n, self.m,
                                     lh.TILED[self.dtype] if self.tiled else self.dtype)


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

    def step(self, ctx, i):
        super().step(ctx, i)
        lh.check(lh.lib().lg_dispatch_argmax(self.c.ptr, self.n, self.m, self.n, self.idx.ptr, ctx.stream))


class DFlashBlock(Workload):
    """The 6-layer draft decoder's block forward: 16 tokens over a 2048-position f32
    K/V context, random-init weights (Q4_K except Q8_0 attn_output), replayed as a
    captured HIP graph.  One forward reads every weight once (917 MB > the 256 MB
    Infinity Cache), so a single model copy needs no rotation."""

    def __init__(self, m=16, ctx_len=2048, seed=0x5EED000A, graph=True):
        self.m, self.ctx_len, self.seed, self.graph_mode = m, ctx_len, seed, graph
        self.cfg = lh.DFlashConfig()
        self.k, self.n = self.cfg.n_embd, self.cfg.n_embd
        self.name = (f"DFlash 6-layer block forward, {m} tokens over {ctx_len}-position f32 KV "
                     f"({'HIP graph' if graph else 'eager'})")

    def setup(self, ctx):
        cfg, m = self.cfg, self.m
        W, layers = synth.dflash_model(self.seed, cfg, cfg.n_layers)
        feat, tok, kc, vc = synth.dflash_inputs(self.seed + 1, cfg, cfg.n_layers, m, self.ctx_len)
        nbytes = lambda a: np.asarray(a).nbytes
        wbytes = sum(nbytes(W[n]) for n in ("enc_aux_norm", "fc", "enc_output_norm", "output_norm"))
        wbytes += sum(nbytes(L[n]) for L in layers for n in lh.DFLASH_NORMS + lh.DFLASH_PROJ)
        kvbytes = sum(nbytes(a) for a in kc + vc)
        self.bytes_per_call = wbytes + kvbytes + feat.nbytes + tok.nbytes + 4 * m * cfg.n_embd
        self.model = lh.DFlashModel(ctx, cfg, W, layers)
        self.model.set_context(kc, vc)
        del W, layers, kc, vc
        self.fb, self.tb = lh.upload_f32(ctx, feat), lh.upload_f32(ctx, tok)
        self.ob = lh.GpuBuffer(ctx, 4 * m * cfg.n_embd)
        self.stream = lh.Stream()
        self.g = self.model.capture(self.fb, self.tb, m, self.ob, self.stream) if self.graph_mode else None
        self.pool = [self.fb, self.tb, self.ob]
        self.pool_bytes = self.bytes_per_call

    def step(self, ctx, i):
        if self.g is not None:
            self.g.launch()
        else:
            self.model.forward_block_device(self.fb, self.tb, self.m, self.ob, stream=self.stream)

    def teardown(self):
        if self.g is not None:
            self.g.destroy()
        self.model.free()
        self.stream.sync()


WORKLOADS = {
    "q4k_m1": lambda: MatvecM1(lh.Q4_K, 4096, 14336, 0x5EED0003),
    "q8_0_m1": lambda: MatvecM1(lh.Q8_0, 4096, 4096, 0x5EED0001),
    "q4k_down_silu": lambda: MatvecM1(lh.Q4_K, 14336, 4096, 0x5EED0005, fused=True),
    "q4k_m16_bf16": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.BF16, 0x5EED0008),
    "q4k_m16_f32": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.F32, 0x5EED0008),
    "q4k_m16_f32_tiled": lambda: BatchM16(lh.Q4_K, 4096, 14336, lh.F32, 0x5EED0008, tiled=True),
    "q8_0_m16_f32": lambda: BatchM16(lh.Q8_0, 4096, 4096, lh.F32, 0x5EED0009),
    "q8_0_m16_f32_tiled": lambda: BatchM16(lh.Q8_0, 4096, 4096, lh.F32, 0x5EED0009, tiled=True),
    # vocab-sized output projection (the LM head, src/target.rs:580-605): M=1 for one
    # token, M=16 to verify a 16-token draft block
    "q4k_lm_head_m1": lambda: MatvecM1(lh.Q4_K, 4096, 151936, 0x5EED000B),
    "q4k_lm_head_m16": lambda: BatchM16(lh.Q4_K, 4096, 151936, lh.F32, 0x5EED000B),
    "lm_head_verify_m16": lambda: VerifyBlock(4096, 151936, 0x5EED000B),
    "dflash_block": lambda: DFlashBlock(),
    "dflash_block_eager": lambda: DFlashBlock(graph=False),
}


def time_workload(ctx, ev, wl, steps, warmup):
    wl.setup(ctx)
    stream = wl.stream.ptr if getattr(wl, "stream", None) is not None else ctx.stream
    sync = wl.stream.sync if getattr(wl, "stream", None) is not None else ctx.sync
    for i in range(warmup):
        wl.step(ctx, i)
    sync()
    a, b = ev.new(), ev.new()
    t0 = time.perf_counter()
    ev.record(a, stream)
    for i in range(steps):
        wl.step(ctx, warmup + i)
    ev.record(b, stream)
    sync()
    wall = time.perf_counter() - t0
    ms = ev.elapsed_ms(a, b)
    us = 1000.0 * ms / steps
    gbs = wl.bytes_per_call / (us * 1e-6) / 1e9
    for p in wl.pool:
        p.free()
    wl.pool = []
    if hasattr(wl, "teardown"):
        wl.teardown()
    r = {"workload": wl.name, "us_per_call": round(us, 3), "GBps": round(gbs, 1),
         "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_call": wl.bytes_per_call,
         "pool_MB": round(wl.pool_bytes / 2 ** 20, 1), "host_wall_s": round(wall, 4)}
    if isinstance(wl, DFlashBlock):
        r["draft_tokens_per_s"] = round(wl.m / (us * 1e-6), 1)
    return r


def cpu_baseline(budget_s=12.0):
    """The oracle's proj_q4k.comp-order matvec (per-element decode, f32 accumulation)
    on the host cores, on the same 4096 -> 14336 Q4_K workload: the whole matvec
    repeated on `threads` OpenMP threads for about budget_s/2 seconds, and a
    bounded sample of output rows on one thread for the other half."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc

    k, n = 4096, 14336
    threads = max(1, min(16, os.cpu_count() or 1))
    raw = synth.q4k_weight(0x5EED0003, k, n)
    x = synth.normal(0x5EED0004, k)
    bytes_per_row = (k // 256) * 144 + 4
    # multi-threaded: whole matvecs
    reps, t_mt = 0, 0.0
    while t_mt < budget_s / 2 or reps < 2:
        t0 = time.perf_counter()
        orc.proj_q4k(x, raw, k, n, threads=threads)
        t_mt += time.perf_counter() - t0
        reps += 1
    gbs_mt = reps * (n * bytes_per_row + 4 * k) / t_mt / 1e9
    # single thread: consecutive 512-row blocks (wrapping) until the budget is spent
    rows, t_st = 0, 0.0
    while t_st < budget_s / 2:
        r0 = rows % n
        r = min(512, n - r0)
        sub = raw[r0 * (k // 256) * 144:(r0 + r) * (k // 256) * 144]
        t0 = time.perf_counter()
        orc.proj_q4k(x, sub, k, r, threads=1)
        t_st += time.perf_counter() - t0
        rows += r
    gbs_st = (rows * bytes_per_row + 4 * k) / t_st / 1e9
    return {"value": round(gbs_mt, 3), "unit": "GB/s", "cores": threads, "kind": "port",
            "single_thread_GBps": round(gbs_st, 4),
            "sample": f"oracle restatement of kernels/proj_q4k.comp (f32 per-element decode) on Q4_K "
                      f"4096->14336 M=1: {reps} full matvecs on {threads} threads in {t_mt:.1f} s; "
                      f"single thread {rows} rows in {t_st:.1f} s"}


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
    wl.setup(ctx)
    for i in range(steps):
        wl.step(ctx, i)
    ctx.sync()
    print(json.dumps({"pmc_run": wl.name, "steps": steps, "calibration_copy_bytes": CAL_BYTES}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
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
    ev = HipEvents()
    wl = WORKLOADS[args.workload]()
    head = time_workload(ctx, ev, wl, args.steps, args.warmup)
    extra = {}
    if not args.no_extra:
        for name in ["q8_0_m1", "q4k_down_silu", "q4k_m16_bf16", "q4k_m16_f32", "q4k_m16_f32_tiled", "q8_0_m16_f32",
                     "q8_0_m16_f32_tiled", "q4k_lm_head_m1", "q4k_lm_head_m16", "lm_head_verify_m16"]:
            if name != args.workload:
                extra[name] = time_workload(ctx, ev, WORKLOADS[name](), max(50, args.steps // 4), 20)
        for name in ["dflash_block", "dflash_block_eager"]:
            if name != args.workload:
                extra[name] = time_workload(ctx, ev, WORKLOADS[name](), max(10, args.steps // 40), 3)
    line = {
        "metric": METRIC,
        "value": head["GBps"],
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
        "config": {"workload": head["workload"], "k": wl.k, "n": wl.n, "m": getattr(wl, "m", 1),
                   "weight_pool_MB": head["pool_MB"], "parallelism": "single GPU"},
        "roofline": {"bound": "hbm", "achieved": head["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": head["frac_of_peak"], "traffic": traffic_from_profile(args.workload),
                     "us_per_call": head["us_per_call"], "algorithmic_bytes": head["bytes_per_call"]},
        "extra": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
