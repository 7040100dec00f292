"""Per-wavefront phase timestamps of the small-M product and the draft attention kernels.

Measurement only: this builds an instrumented copy of the library in which lane 0 of
every wavefront writes the real-time clock (s_memrealtime, 100 MHz) at the phase
boundaries listed in STAMPS, plus the hardware CU it runs on, into a device array; then
it runs a bench.py workload and prints, per stamp, percentiles over the wavefronts of the
last call (ns from the first wavefront's start), and how the workgroups spread over CUs.
The shipped library is not touched; the instrumented one is built into _timeline/
(each wavefront's lane 0 stores its stamps with ordinary vector stores).

    python timeline.py build [--tiles] [--mm-if CONDITION]
    python timeline.py run WORKLOAD [mm|attn]

`--mm-if` keeps the small-M product's stamps to the instances whose template parameters
satisfy CONDITION (C++ over Q4, TT, RT, GLU, NORM, TILED, XM; e.g. "NORM && !GLU", the draft's
K/V/Q launch), so that `run ... mm` reads that launch rather than the workload's last product.

`--tiles` adds stamps inside the attention's tile loop (after each tile's scores and
after its P V, each with the next tile's loads issued); they slow that kernel by about
a quarter, so its other phases read best from a build without them.

`mm` reads the last small-M product launch (k_mm_mf) of the workload, `attn` the last k_attn_split launch
(the draft block's last layer), or the last combine launch of the few-query path, `m1` the last launch of
the M = 1 integer-dot Q4_K kernel (k_q4k_m1_dig and its norm-fused forms).
"""
import argparse
import collections
import ctypes
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_timeline")
LIB = os.path.join(OUT, "liblaguna_hip_timeline.so")
HIPCC = "/opt/rocm/bin/hipcc"
SLOTS, WAVES = 40, 6553  # stamps per wavefront, wavefronts recorded

HEADER = r'''
__device__ unsigned long long lg_tl_%(f)s[%(n)d];
extern "C" int lg_timeline_read_%(f)s(void *host, unsigned long long bytes) {
    return hipMemcpyFromSymbol(host, HIP_SYMBOL(lg_tl_%(f)s), bytes) == hipSuccess ? 0 : 1;
}
extern "C" int lg_timeline_clear_%(f)s() {
    static unsigned long long z[%(n)d];
    return hipMemcpyToSymbol(HIP_SYMBOL(lg_tl_%(f)s), z, sizeof(z)) == hipSuccess ? 0 : 1;
}
#define LG_WID() (((blockIdx.y * gridDim.x) + blockIdx.x) * (blockDim.x >> 6) + (threadIdx.x >> 6))
#define TS(k) do { if constexpr (%(cond)s) { const unsigned long long t_ = __builtin_amdgcn_s_memrealtime(); \
    if ((threadIdx.x & 63u) == 0 && LG_WID() < %(w)du) lg_tl_%(f)s[LG_WID() * %(s)d + (k)] = t_; } } while (0)
#define TSID() do { if constexpr (%(cond)s) { unsigned hw_, xc_; \
    asm volatile("s_getreg_b32 %%0, hwreg(HW_REG_HW_ID)" : "=s"(hw_)); \
    asm volatile("s_getreg_b32 %%0, hwreg(HW_REG_XCC_ID)" : "=s"(xc_)); \
    if ((threadIdx.x & 63u) == 0 && LG_WID() < %(w)du) \
        lg_tl_%(f)s[LG_WID() * %(s)d + %(s)d - 1] = ((unsigned long long)xc_ << 32) | hw_; } } while (0)
'''

# (file, kernel signature start, [(mode, marker, text)]): text goes after / before the
# first occurrence of marker past the kernel's start.
STAMPS = {
    "proj_batch.hip": ("void mm_body(", [
        ("after", "lg_u32x4 *lstage) {", "\n    TS(0); TSID();"),
        ("after", "    rb.store(lrec[0], m);\n    __syncthreads();", "\n    TS(1);"),
        ("after", "            rb.store(lrec[c & 1u], m);\n            __syncthreads();",
         "\n            if (c < 34) TS(1 + c);"),
        ("before", "    static_assert(!GLU || 2 * RT * TT * 256 * 4", "    TS(36);\n"),
        ("after", "jobs.j[J_].y, jobs.j[J_].yw, jobs.j[J_].ss, bx, jobs.j[J_].qkw);", "\n    TS(38);"),
    ]),
    "dflash.hip": ("void k_attn_split(", [
        ("after", "grp = h * a.ngq + qg;", "\n    TS(0); TSID();"),
        ("before", "    const uint32_t nt = (a.S + 15) / 16, tb = attn_tile0(c, nt, a.nch)", "    TS(1);\n"),
        ("before", "        for (uint32_t i = 0; i < nmine; i += 2) {", "        TS(2);\n"),
        ("before", "    lsum = lane_add_x32(lane_add_x16(lsum));", "    TS(3);\n"),
        ("before", "    // thread (query mq, dims md .. md + ", "    TS(4);\n"),
        ("before", "    // the last workgroup of the group to arrive merges", "    TS(5);\n"),
        ("after", "if (!arrive_last(a.cnt + grp, a.nch, &last)) return;", "\n    TS(6);"),
        ("before", "    const uint32_t qo = AQG * qg + mq;", "    TS(7);\n"),
    ]),
    "proj_m1.hip": ("void q4k_m1_dig_body(", [
        ("after", "    const uint32_t stride = gridDim.x * TEAMS * R;\n", "    TS(0); TSID();\n"),
        ("after", "    dig_convert(xv, k, dg);\n    __syncthreads();", "\n    TS(1);"),
        ("after", "    dig_read(dg, p, D, X0, X1, F);", "\n    TS(2);"),
        ("before", "    auto reduce = [&](int b, uint32_t rr) {", "    uint32_t tl_n = 0;\n"),
        ("after", "            float v = dotrow(hd[b][r], qa[b][r], qb[b][r]);",
         "\n            if (r == 0) { if (tl_n < 30) TS(3 + tl_n); tl_n++; }"),
        ("after", "        r0 = r2;\n    }", "\n    TS(38);"),
    ]),
    "dflash.hip#combine": ("void k_attn_combine(", [
        ("after", "if (h >= n_kv || qi >= rows * G) return;  // uniform over the workgroup", "\n    TS(20);"),
        ("before", "    float M = tm, L = tl, o0 = t0, o1 = t1;", "    TS(21);\n"),
        ("before", "    if (lane == 0) sm[wave] = M, sl[wave] = L;", "    TS(22);\n"),
        ("before", "    const float Mx = fmaxf", "    TS(23);\n"),
        ("before", "    const float inv = L > 0.0f ? 1.0f / L : 0.0f;", "    TS(24);\n"),
    ]),
}

# the attention's per-tile stamps (build --tiles): slot 8 + 2i after tile i's scores and
# K loads, 9 + 2i after its P V and V loads
TILE_STAMPS = [
    ("before", "    auto tile_step = [&]", "    uint32_t tl_i = 0;\n"),
    ("after", "        load_k(kr, next);\n        __builtin_amdgcn_sched_barrier(0);",
     "\n        if (tl_i < 6) TS(8 + 2 * tl_i);"),
    ("after", "        load_v(vr, next);\n        __builtin_amdgcn_sched_barrier(0);",
     "\n        if (tl_i < 6) TS(9 + 2 * tl_i);\n        tl_i++;"),
]

PHASES = {
    "mm": [(0, "start"), (1, "chunk 0's activations in LDS"), (2, "chunk 1 in LDS"), (3, "chunk 2 in LDS"),
           (4, "chunk 3 in LDS"), (36, "products done"), (38, "split-k finish done")],
    "m1": [(0, "start"), (1, "x converted (after the barrier)"), (2, "digits in registers"),
           (3, "first rows reduced"), (4, "second rows"), (5, "third rows"), (6, "fourth rows"), (38, "done")],
    "attn": [(0, "start"), (1, "queries issued"), (2, "first tile issued, gate units done"),
             (8, "tile 0: scores, K refill issued"), (9, "tile 0: P V, V refill issued"),
             (10, "tile 1: scores"), (11, "tile 1: P V"), (12, "tile 2: scores"), (13, "tile 2: P V"),
             (14, "tile 3: scores"), (15, "tile 3: P V"), (16, "tile 4: scores"), (17, "tile 4: P V"),
             (3, "tiles done"), (4, "wavefronts met in LDS"), (5, "partial stored"), (6, "last to arrive"),
             (7, "chunks merged"), (20, "combine: start"), (21, "tail / gate"), (22, "chunk partials merged"),
             (23, "waves met in LDS"), (24, "result")],
}


def instrument(src, sig, edits):
    s = src
    k0 = s.index(sig)
    for mode, marker, text in edits:
        j = s.index(marker, k0)
        j = j + len(marker) if mode == "after" else j
        s = s[:j] + text + s[j:]
    return s


def build(tiles=False, mm_if="true"):
    os.makedirs(OUT, exist_ok=True)
    csrc = os.path.join(HERE, "csrc")
    flags = ["-x", "hip", "--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature",
             "-Xclang", "-packed-fp32-ops", "-I" + os.path.join(HERE, "..", "include"), "-I" + csrc]
    ilp = ["-mllvm", "-amdgpu-mfma-vgpr-form", "-mllvm", "-amdgpu-sched-strategy=max-ilp"]
    extra = {"proj_batch.hip": ilp, "dflash.hip": ilp,
             "proj_m1.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"]}
    objs = []
    for f in ["runtime.cpp", "gguf.cpp", "dequant.hip", "proj_m1.hip", "proj_batch.hip", "dflash.hip", "verify.hip",
              "ceiling.hip", "target.hip"]:
        src = open(os.path.join(csrc, f)).read()
        if f in ("proj_batch.hip", "dflash.hip", "proj_m1.hip"):
            for key, (sig, edits) in STAMPS.items():
                if key.split("#")[0] == f:
                    src = instrument(src, sig, edits + (TILE_STAMPS if tiles and key == "dflash.hip" else []))
            i = src.index("namespace {")
            tag = {"proj_batch.hip": "mm", "dflash.hip": "attn", "proj_m1.hip": "m1"}[f]
            cond = mm_if if tag == "mm" else "true"
            src = src[:i] + HEADER % {"f": tag, "n": SLOTS * WAVES, "w": WAVES, "s": SLOTS, "cond": cond} + src[i:]
        path = os.path.join(OUT, f)
        open(path, "w").write(src)
        obj = path + ".o"
        subprocess.run([HIPCC] + flags + extra.get(f, []) + ["-c", path, "-o", obj], check=True)
        objs.append(obj)
    subprocess.run([HIPCC, "--offload-arch=gfx950", "-shared", "-o", LIB] + objs, check=True)
    print("built", LIB)


def run(workload, what, dump=None):
    sys.path.insert(0, HERE)
    sys.path.insert(0, os.path.join(HERE, ".."))
    import numpy as np
    import laguna_hip as lh
    lh.LIB_PATH = LIB
    import bench
    L = lh.lib()
    read = getattr(L, "lg_timeline_read_" + what)
    read.argtypes = [ctypes.c_void_p, ctypes.c_ulonglong]
    ctx = lh.VulkanContext(0)
    wl = bench.WORKLOADS[workload]()
    st = lh.Stream()
    if isinstance(wl, bench.DFlashBlock):
        wl.setup(ctx, st)
    else:
        wl.setup(ctx)
    for i in range(10):
        wl.step(i, st.ptr)
    st.sync()
    lh.check(getattr(L, "lg_timeline_clear_" + what)())
    ctx.sync()
    for i in range(3):  # stamps of the last call survive
        wl.step(100 + i, st.ptr)
    st.sync()
    buf = np.zeros(SLOTS * WAVES, np.uint64)
    lh.check(read(buf.ctypes.data, buf.nbytes))
    ts = buf.reshape(WAVES, SLOTS)
    if dump:
        np.save(dump, ts)
    live = (ts[:, 0] > 0) | (ts[:, 20] > 0)
    n = int(np.nonzero(live)[0].max()) + 1
    T = ts[:n, :SLOTS - 1].astype(np.int64)
    starts = [T[:, k][T[:, k] > 0] for k in (0, 20)]
    t0 = min(v.min() for v in starts if v.size)
    print(f"{workload} ({what}): {n} wavefronts of the last call; ns from the first wavefront's start")
    print("| stamp | phase | p10 | p50 | p90 | max |")
    print("|---|---|---|---|---|---|")
    for k, name in PHASES[what]:
        v = T[:, k]
        v = (v[v >= t0] - t0) * 10  # stamps of the last launch only (others are left from earlier ones)
        if v.size:
            print(f"| {k} | {name} | {int(np.percentile(v, 10))} | {int(np.median(v))} | "
                  f"{int(np.percentile(v, 90))} | {int(v.max())} |")
    nw = int(np.nonzero(ts[:, 0] > 0)[0].max()) + 1  # wavefronts of the kernel that records its CU
    ids = ts[:nw, SLOTS - 1]
    hw, xcc = ids & 0xFFFFFFFF, ids >> 32
    # HW_ID: CU_ID bits 8-11, SH_ID bit 12, SE_ID bits 13-15 (gfx9)
    cu = (xcc << 8) | (((hw >> 13) & 7) << 5) | (((hw >> 12) & 1) << 4) | ((hw >> 8) & 15)
    wpg = 4
    wg_cu = cu[0::wpg]
    rel = np.where(T[:nw] > 0, (T[:nw] - t0) * 10, -1)
    end_k = 5 if what == "attn" else 38
    ends = rel[:, end_k].reshape(-1, wpg).max(axis=1)
    wg_xcc = xcc[0::wpg]
    rr = int((wg_xcc == (np.arange(len(wg_xcc)) % 8)).sum())
    print(f"workgroups on XCD (workgroup id mod 8): {rr} of {len(wg_xcc)}")
    cnt = collections.Counter(wg_cu.tolist())
    hist = collections.Counter(cnt.values())
    print(f"\nworkgroups {len(wg_cu)} on {len(cnt)} CUs; CUs by workgroups held: {dict(sorted(hist.items()))}")
    for c in sorted(hist):
        sel = np.array([cnt[x] == c for x in wg_cu.tolist()])
        e = ends[sel]
        e = e[e >= 0]
        if e.size:
            print(f"workgroups on CUs holding {c}: {int(sel.sum())}, end p50 {int(np.median(e))} ns, "
                  f"max {int(e.max())} ns")
    wl.teardown()


def main():
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    b = sub.add_parser("build")
    b.add_argument("--tiles", action="store_true")
    b.add_argument("--mm-if", default="true")
    r = sub.add_parser("run")
    r.add_argument("workload")
    r.add_argument("what", nargs="?", default="mm", choices=["mm", "attn", "m1"])
    r.add_argument("--dump", help="also save the raw stamps (wavefronts x slots, .npy)")
    a = ap.parse_args()
    build(a.tiles, a.mm_if) if a.cmd == "build" else run(a.workload, a.what, a.dump)


if __name__ == "__main__":
    main()
