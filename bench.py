#!/usr/bin/env python3
"""Benchmark of the MXFP4 hot path on one MI355X.

A step is one BF16 -> MXFP4 rowwise quantize of the 8192 x 7168 activation
tensor (N(0,1), 0.1% of the channels x100), launched through the C ABI
(omo_hip_per_token_group_quant_fp4) on torch's current HIP stream. Inputs are
resident in HBM before the timed region. Four input/output buffer sets
(594 MB) rotate so that the 256 MB Infinity Cache cannot hold the working
set. The script prints one JSON line.

Also measured (extra keys): MXFP4 -> BF16 dequant of the same shape, the
cfg1 quantize + dequantize round trip (4096 x 4096), the MoE-payload requant/dequant (4096 x 7168, both FP8 layouts), the fused
expert-parallel payload rows against Megatron's cat/split composition, the
MXFP4 moe_permute gather (alone and fused into the FP8 requant), the
cfg5 MoE layer composite (all codec launches of one layer on 8 local experts),
the dual-layout quantize (7168 x 18432), the row -> col FP8 conversion and
the per-split row -> col FP8 of cfg5's routed rows alone, each as GB/s of algorithmic bytes or microseconds per call, and memory-only
kernels over the headline buffers (the quantize's loads and stores without
its arithmetic; streaming reads; streaming writes) as the practical bound.
On request only (--only floors): each bandwidth-bound codec kernel beside a
memory-only copy of its own access pattern, the floor that pattern sets.

The CPU baseline runs the oracle (a multithreaded C restatement of the
reference kernels) on the host's cores for the headline quantize and, in the
legs that have one, for cfg1's round trip, the cfg2 dequant and cfg4's FP8
requant and dequant; each of those also checks the GPU outputs against it.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       [--only headline|dequant,cfg1,...] [--copy-calibration]
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "mxfp4-hopper_amd"))

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published peak
METRIC = "BF16→MXFP4 quantize GB/s & % HBM peak at 8192×7168; dequant GB/s"


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--sets", type=int, default=4, help="rotating buffer sets (>= 3 to exceed the 256 MB cache)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", default="",
                    help="comma list of extra legs: dequant,cfg1,payload,ep_payload,permute,moe,msplit,dual,rowcol,"
                         "rowcol_partial,"
                         "ceiling,floors ('floors' runs only when named); 'headline' runs the headline "
                         "quantize alone")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 1 GiB device copy (known traffic) for counter calibration")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--eager", action="store_true",
                    help="time eagerly enqueued launches only (no HIP graph), e.g. under counter collection")
    return ap.parse_args()


def sleep_gpu(torch, ms=5.0):
    """Keep the GPU busy while the host enqueues the timed launches, so the
    timed region measures the GPU rather than the host's enqueue rate."""
    try:
        torch.cuda._sleep(int(ms * 2.4e6))
    except Exception:
        pass


GRAPH = True


def _split_meta(m_splits):
    """Exclusive prefix sums of the grouped row -> col kernel: (lens, row
    offsets, scale-row offsets, max split length)."""
    offs, soffs, o, so = [], [], 0, 0
    for m in m_splits:
        offs.append(o)
        soffs.append(so)
        o += m
        so += -(-m // 128)
    return list(m_splits), offs, soffs, max(m_splits) if m_splits else 0


def cpu_model():
    """The host CPU's model name (Linux), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_threads():
    """Threads for the CPU baseline and what bounds them. The oracle runs on
    every CPU this process may use (its affinity mask), capped by the cgroup
    CPU quota and by OMP_NUM_THREADS where the host sets them: on a shared GPU
    host those state this GPU's share of the cores. Returns (threads, info)."""
    info = {"host_logical_cpus": os.cpu_count()}
    try:
        aff = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        aff = os.cpu_count() or 1
    info["affinity_cpus"] = aff
    n = aff
    quota = None
    try:
        with open("/sys/fs/cgroup/cpu.max") as f:
            q, period = f.read().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(period))
    except (OSError, ValueError):
        pass
    info["cgroup_cpu_quota"] = quota
    if quota:
        n = min(n, quota)
    omp = os.environ.get("OMP_NUM_THREADS", "")
    info["omp_num_threads"] = int(omp) if omp.isdigit() and int(omp) > 0 else None
    if info["omp_num_threads"]:
        n = min(n, info["omp_num_threads"])
    info["threads_used"] = n
    return n, info


def cpu_time(fn, seconds, min_reps=3, max_reps=2000):
    """Runs fn repeatedly for about `seconds` (at least min_reps times);
    returns (last result, median seconds per call, reps, total seconds)."""
    times = []
    res = None
    t_end = time.time() + seconds
    while len(times) < min_reps or (time.time() < t_end and len(times) < max_reps):
        t0 = time.perf_counter()
        res = fn()
        times.append(time.perf_counter() - t0)
    return res, statistics.median(times), len(times), sum(times)


def sets_for(bytes_per_set, minimum):
    """Buffer sets to rotate so the working set exceeds 512 MB, twice the
    256 MB Infinity Cache."""
    return max(minimum, -(-512_000_000 // bytes_per_set))


def time_launches(torch, launch, n_sets, steps, warmup, graph=None):
    """Warm up, then time exactly `steps` back-to-back launches (rotating over
    the buffer sets) with one HIP event at each end of the timed region, on the
    stream the kernels run on. With graph=True the `steps` launches are first
    captured into one HIP graph, whose single replay is the timed region.
    Returns (total_ms, eager_total_ms)."""
    for i in range(warmup):
        launch(i % n_sets)
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    sleep_gpu(torch)
    t0.record()
    for i in range(steps):
        launch(i % n_sets)
    t1.record()
    torch.cuda.synchronize()
    eager = t0.elapsed_time(t1)
    if not (GRAPH if graph is None else graph):
        return eager, eager
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                launch(i % n_sets)
    torch.cuda.current_stream().wait_stream(s)
    g.replay()  # untimed warm replay
    torch.cuda.synchronize()
    t0.record()
    g.replay()
    t1.record()
    torch.cuda.synchronize()
    total = t0.elapsed_time(t1)
    del g
    return total, eager


def ceiling_leg(torch, args, dev, cur, xs, qs, ss, numel, qbytes, value):
    """Memory-only kernels at the headline size: the quantize's loads and
    stores without its arithmetic (one-pass and two-phase schedules), and
    pure streaming reads / writes."""
    import ctypes
    cl = ctypes.CDLL(os.path.join(ROOT, "mxfp4-hopper_amd", "lib", "libomo_ceiling.so"))
    cl.omo_ceiling_launch.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_int64, ctypes.c_void_p]
    n16 = numel * 2 // 16
    wbuf = [torch.empty(n16 * 16, dtype=torch.uint8, device=dev) for _ in range(args.sets)]
    res = {}
    for kind, name, nbytes in ((0, "quant_traffic", qbytes), (3, "two_phase_traffic", qbytes),
                               (1, "read_stream", n16 * 16), (2, "write_stream", n16 * 16)):
        def mem(i, kind=kind):
            dst = wbuf[i] if kind == 2 else qs[i]
            rc = cl.omo_ceiling_launch(kind, xs[i].data_ptr(), dst.data_ptr(), ss[i].data_ptr(), n16, cur())
            if rc:
                raise RuntimeError(f"omo_ceiling_launch({kind}) returned {rc}")
        steps = max(100, args.steps // 2)
        t, _ = time_launches(torch, mem, args.sets, steps, 20)
        res[name] = (round(nbytes / (t / steps * 1e-3) / 1e9, 1), round(t / steps * 1e3, 3))
    best = max(res["quant_traffic"][0], res["two_phase_traffic"][0])
    return {
        "workload": "memory-only kernels over the 8192x7168 headline buffers (mxfp4-hopper_amd/ceiling)",
        "quant_traffic_GB/s": res["quant_traffic"][0], "quant_traffic_us": res["quant_traffic"][1],
        "two_phase_traffic_GB/s": res["two_phase_traffic"][0], "two_phase_traffic_us": res["two_phase_traffic"][1],
        "quant_frac_of_ceiling": round(value / best, 4),
        "read_stream_GB/s": res["read_stream"][0], "write_stream_GB/s": res["write_stream"][0]}


def floors_leg(torch, args, dev, cur, lib, _abi, wl):
    """Each bandwidth-bound codec kernel beside a memory-only copy of its own
    access pattern (mxfp4-hopper_amd/ceiling/mem_floors.hip: the same loads,
    stores, workgroup shape, order and LDS footprint, no arithmetic), on the
    same buffers: the floor that pattern sets on this HBM. Beside them,
    memory-only copies of schedules the product does not use (alt): what a
    different schedule of the same traffic would allow."""
    import ctypes
    fl = ctypes.CDLL(os.path.join(ROOT, "mxfp4-hopper_amd", "lib", "libomo_ceiling.so"))
    P, I64 = ctypes.c_void_p, ctypes.c_int64
    fl.omo_floor_dual.argtypes = [P, P, P, P, P, I64, I64, P]
    fl.omo_floor_rowcol.argtypes = [P, P, P, P, I64, I64, P]
    fl.omo_floor_msplit.argtypes = [P, P, P, P, I64, I64, P, P, P, I64, I64, I64, P]
    fl.omo_floor_requant.argtypes = [P, P, P, P, I64, I64, P]
    fl.omo_floor_dequant.argtypes = [P, P, P, I64, P]
    fl.omo_floor_dual_variant.argtypes = [ctypes.c_int, P, P, P, P, P, I64, I64, P]
    fl.omo_floor_msplit_band.argtypes = [P, P, P, P, I64, P, P, P, I64, I64, P]
    fl.omo_floor_dual_grouped.argtypes = [ctypes.c_int, P, P, P, P, P, P, P, ctypes.c_int, P]

    def chk(rc, what):
        if rc:
            raise RuntimeError(f"{what} returned {rc}")

    def pair(name, workload, nbytes, n_sets, product, floor, steps):
        tp, _ = time_launches(torch, product, n_sets, steps, 10)
        tf, _ = time_launches(torch, floor, n_sets, steps, 10)
        up, uf = tp / steps * 1e3, tf / steps * 1e3
        res[name] = {"workload": workload, "kernel_us": round(up, 2), "floor_us": round(uf, 2),
                     "kernel_frac_of_floor": round(uf / up, 3), "floor_frac_of_peak": round(nbytes / (uf * 1e-6) / 8e12, 3)}

    def alt(name, workload, nbytes, n_sets, floor, steps, against):
        """A memory-only copy of a schedule the product does not use, timed on
        the same buffers as `against`'s pair."""
        tf, _ = time_launches(torch, floor, n_sets, steps, 10)
        uf = tf / steps * 1e3
        res[name] = {"workload": workload, "floor_us": round(uf, 2),
                     "floor_frac_of_peak": round(nbytes / (uf * 1e-6) / 8e12, 3),
                     "vs_product_floor": round(res[against]["floor_us"] / uf, 3)}

    res = {}
    # dual-layout quantize, cfg3 7168 x 18432
    M, K = 7168, 18432
    n = M * K
    xd = [wl.heavy_tail_weights(M, K, seed=33 + i, device=dev) for i in range(2)]
    od = [[torch.empty(b, dtype=torch.uint8, device=dev) for b in (n // 2, n // 32, n // 2, n // 32)] for _ in range(2)]
    pair("dual", "dual-layout quantize 7168x18432 (quant_dual_super_kernel)", wl.dual_quant_bytes(n), 2,
         lambda i: chk(lib.omo_hip_quant_mxfp4_dual(xd[i].data_ptr(), M, K, od[i][0].data_ptr(), n // 2,
                                                    od[i][1].data_ptr(), n // 32, od[i][2].data_ptr(), n // 2,
                                                    od[i][3].data_ptr(), n // 32, 1e-10, cur()), "dual"),
         lambda i: chk(fl.omo_floor_dual(xd[i].data_ptr(), od[i][0].data_ptr(), od[i][1].data_ptr(),
                                         od[i][2].data_ptr(), od[i][3].data_ptr(), M, K, cur()), "dual floor"),
         max(20, args.steps // 50))
    for kind, name, what in ((1, "dual_no_scale_stores", "the product's schedule without its scale stores (the bound "
                                                         "of the code traffic; not a valid output)"),
                             (2, "dual_scales_as_whole_lines", "the product's schedule with each workgroup's 4 KB of "
                                                               "scale bytes stored as whole non-temporal lines "
                                                               "(layout-free bound; not a valid output)"),
                             (3, "dual_k_fastest", "the product's stores in contiguous K-fastest super-tile "
                                                   "ranges per XCD"),
                             (4, "dual_m_fastest_ranges", "the product's stores in contiguous M-fastest super-tile "
                                                          "ranges per XCD (each XCD finishing a band before the "
                                                          "next)"),
                             (5, "dual_aligned_groups", "the product's stores with each XCD owning whole 8-band "
                                                        "groups (64 B halves of the row-scale lines) and an eighth "
                                                        "of the leftover groups")):
        alt(name, f"dual-layout floor 7168x18432: {what}", wl.dual_quant_bytes(n), 2,
            lambda i, kind=kind: chk(fl.omo_floor_dual_variant(kind, xd[i].data_ptr(), od[i][0].data_ptr(),
                                                               od[i][1].data_ptr(), od[i][2].data_ptr(),
                                                               od[i][3].data_ptr(), M, K, cur()), "dual variant"),
            max(20, args.steps // 50), "dual")
    del xd, od
    # the grouped dual-layout quantize of cfg5's 24 expert weights (one-tile pattern)
    c5 = wl.CFG5
    w_shapes = [(c5["hidden"], c5["ffn"]), (c5["hidden"], c5["ffn"]), (c5["ffn"], c5["hidden"])] * c5["local_experts"]
    nwi = len(w_shapes)
    bg = sum(wl.dual_quant_bytes(r * c) for r, c in w_shapes)
    gx = [[wl.normal_bf16(sh, seed=100 + i + 50 * si, device=dev, std=0.02) for i, sh in enumerate(w_shapes)]
          for si in range(2)]
    go = [[[torch.empty(b, dtype=torch.uint8, device=dev) for b in (r * c // 2, r * c // 32, r * c // 2, r * c // 32)]
           for r, c in w_shapes] for _ in range(2)]
    g_items = [(_abi.DualItem * nwi)(*[_abi.DualItem(w.data_ptr(), w.size(0), w.size(1), *(v for t in o for v in
                                                                                         (t.data_ptr(), t.numel())))
                                       for w, o in zip(gx[si], go[si])]) for si in range(2)]
    PA = ctypes.c_void_p * nwi
    g_ptrs = [[PA(*[w.data_ptr() for w in gx[si]])] + [PA(*[o[k].data_ptr() for o in go[si]]) for k in range(4)]
              for si in range(2)]
    g_m = (ctypes.c_int64 * nwi)(*[r for r, _ in w_shapes])
    g_k = (ctypes.c_int64 * nwi)(*[c for _, c in w_shapes])

    def g_floor(i, scm):
        chk(fl.omo_floor_dual_grouped(scm, *g_ptrs[i], g_m, g_k, nwi, cur()), "grouped floor")
    pair("dual_grouped", "grouped dual-layout quantize of cfg5's 24 expert weights (quant_dual_grouped_kernel)", bg, 2,
         lambda i: chk(lib.omo_hip_quant_mxfp4_dual_grouped(g_items[i], nwi, 1e-10, cur()), "grouped"),
         lambda i: g_floor(i, 0), max(10, args.steps // 100))
    alt("dual_grouped_no_scale_stores", "grouped dual-layout floor without its scale stores (the bound of the code "
                                        "traffic; not a valid output)", bg, 2, lambda i: g_floor(i, 1),
        max(10, args.steps // 100), "dual_grouped")
    del gx, go, g_items, g_ptrs
    # the code-reading kernels at cfg4's 4096 x 7168 (dequant at 8192 x 7168)
    M, N = 4096, 7168
    n = M * N
    b4 = wl.requant_fp8_bytes(n)
    ns = sets_for(b4, 4)
    x4 = wl.normal_bf16((M, N), seed=60, device=dev)
    q4 = [torch.empty((M, N // 2), dtype=torch.uint8, device=dev) for _ in range(ns)]
    s4 = [torch.empty((M, N // 32), dtype=torch.uint8, device=dev) for _ in range(ns)]
    for i in range(ns):
        chk(lib.omo_hip_per_token_group_quant_fp4(x4.data_ptr(), n, q4[i].data_ptr(), n // 2, s4[i].data_ptr(),
                                                  n // 32, 32, 1e-10, -6.0, 6.0, 0, cur()), "quantize")
    del x4
    o4 = [torch.empty(n, dtype=torch.uint8, device=dev) for _ in range(ns)]
    os4 = [torch.empty(n // 128, dtype=torch.float32, device=dev) for _ in range(ns)]
    steps = max(100, args.steps // 4)
    pair("requant_fp8", "rowwise FP8 requant 4096x7168 (mxfp4_to_fp8_kernel)", b4, ns,
         lambda i: chk(lib.omo_hip_per_token_Mxfp4ToFp8(q4[i].data_ptr(), M, N // 2, s4[i].data_ptr(), n // 32,
                                                        o4[i].data_ptr(), n, os4[i].data_ptr(), n // 128, 128, 1e-10,
                                                        -6.0, 6.0, 0, cur()), "requant"),
         lambda i: chk(fl.omo_floor_requant(q4[i].data_ptr(), s4[i].data_ptr(), o4[i].data_ptr(), os4[i].data_ptr(), M,
                                            N // 2, cur()), "requant floor"), steps)
    pair("row_to_col_fp8", "row -> col FP8 4096x7168 (row_to_fp8_col_wide_kernel)", wl.row_to_col_fp8_bytes(M, N), ns,
         lambda i: chk(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(q4[i].data_ptr(), M, N // 2, s4[i].data_ptr(), M,
                                                                    N // 32, o4[i].data_ptr(), N, M,
                                                                    os4[i].data_ptr(), M // 128, N, 1e-10, cur()),
                       "row->col"),
         lambda i: chk(fl.omo_floor_rowcol(q4[i].data_ptr(), s4[i].data_ptr(), o4[i].data_ptr(), os4[i].data_ptr(), M, N,
                                           cur()), "row->col floor"), steps)
    del q4, s4, o4, os4
    # per split, cfg5's routed rows
    c5 = wl.CFG5
    m_e = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["local_experts"]), seed=5)
    R, Hd = sum(m_e), c5["hidden"]
    b5 = sum(wl.row_to_col_fp8_bytes(m, Hd) for m in m_e)
    ns = sets_for(b5, 3)
    lens, offs, soffs, mx = (torch.tensor(v, dtype=torch.int32, device=dev) if i < 3 else v
                             for i, v in enumerate(_split_meta(m_e)))
    srows = sum(-(-m // 128) for m in m_e)
    x5 = wl.normal_bf16((R, Hd), seed=70, device=dev)
    q5 = [torch.empty((R, Hd // 2), dtype=torch.uint8, device=dev) for _ in range(ns)]
    s5 = [torch.empty((R, Hd // 32), dtype=torch.uint8, device=dev) for _ in range(ns)]
    for i in range(ns):
        chk(lib.omo_hip_per_token_group_quant_fp4(x5.data_ptr(), R * Hd, q5[i].data_ptr(), R * Hd // 2,
                                                  s5[i].data_ptr(), R * Hd // 32, 32, 1e-10, -6.0, 6.0, 0, cur()),
            "quantize")
    del x5
    o5 = [torch.empty(R * Hd, dtype=torch.uint8, device=dev) for _ in range(ns)]
    os5 = [torch.empty((srows, Hd), dtype=torch.float32, device=dev) for _ in range(ns)]
    pair("msplit", f"per-split row -> col FP8, cfg5's {R} rows in {len(m_e)} ragged splits "
                   "(row_to_fp8_col_msplit_flat_kernel)", b5, ns,
         lambda i: chk(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(
             q5[i].data_ptr(), R, Hd // 2, s5[i].data_ptr(), s5[i].numel(), o5[i].data_ptr(), o5[i].numel(),
             os5[i].data_ptr(), os5[i].numel(), lens.data_ptr(), offs.data_ptr(), soffs.data_ptr(), len(m_e), mx, 1e-10,
             cur()), "msplit"),
         lambda i: chk(fl.omo_floor_msplit(q5[i].data_ptr(), s5[i].data_ptr(), o5[i].data_ptr(), os5[i].data_ptr(), R,
                                           Hd, lens.data_ptr(), offs.data_ptr(), soffs.data_ptr(), len(m_e), mx, srows,
                                           cur()), "msplit floor"), max(50, args.steps // 10))
    alt("msplit_band_schedule", "per-split floor of the band schedule: one workgroup per (split, 64 columns) "
        "staging the split's band in LDS and writing its contiguous [64 x len] output block in address order with "
        "aligned non-temporal 16 B stores", b5, ns,
        lambda i: chk(fl.omo_floor_msplit_band(q5[i].data_ptr(), s5[i].data_ptr(), o5[i].data_ptr(), os5[i].data_ptr(),
                                               Hd, lens.data_ptr(), offs.data_ptr(), soffs.data_ptr(), len(m_e), mx,
                                               cur()), "msplit band floor"), max(50, args.steps // 10), "msplit")
    del q5, s5, o5, os5
    # dequant, 8192 x 7168
    M, N = 8192, 7168
    n = M * N
    bq = wl.dequant_bytes(n)
    ns = sets_for(bq, 4)
    x6 = wl.normal_bf16((M, N), seed=61, device=dev)
    q6 = [torch.empty(n // 2, dtype=torch.uint8, device=dev) for _ in range(ns)]
    s6 = [torch.empty(n // 32, dtype=torch.uint8, device=dev) for _ in range(ns)]
    for i in range(ns):
        chk(lib.omo_hip_per_token_group_quant_fp4(x6.data_ptr(), n, q6[i].data_ptr(), n // 2, s6[i].data_ptr(),
                                                  n // 32, 32, 1e-10, -6.0, 6.0, 0, cur()), "quantize")
    del x6
    y6 = [torch.empty(n, dtype=torch.bfloat16, device=dev) for _ in range(ns)]
    pair("dequant", "dequant 8192x7168 (dequant_bf16_kernel)", bq, ns,
         lambda i: chk(lib.omo_hip_per_token_Mxfp4ToBf16_dequant(q6[i].data_ptr(), n // 2, s6[i].data_ptr(), n // 32,
                                                                y6[i].data_ptr(), n, None, 0, 32, 1e-10, -6.0, 6.0,
                                                                0, cur()), "dequant"),
         lambda i: chk(fl.omo_floor_dequant(q6[i].data_ptr(), s6[i].data_ptr(), y6[i].data_ptr(), n // 8, cur()),
                       "dequant floor"), max(100, args.steps // 4))
    del q6, s6, y6
    res["note"] = ("floor: a memory-only copy of the kernel's own access pattern (mxfp4-hopper_amd/ceiling/"
                   "mem_floors.hip) on the same buffers; kernel_frac_of_floor = floor time / kernel time")
    return res


def main():
    global GRAPH
    args = parse()
    GRAPH = not args.eager
    if args.gpus != 1:
        print(json.dumps({"error": "this build runs on exactly one GPU; --gpus must be 1 "
                          "(the path shards by rows with no exchange; only one GPU is used here)"}))
        sys.exit(2)
    import torch
    import omo
    from omo import _abi
    import omo_workloads as wl

    lib = _abi.lib
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    cur = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    only = set(filter(None, args.only.split(",")))
    want = (lambda leg: not only or leg in only)

    if args.copy_calibration:
        n = 1 << 30
        a = torch.empty(n, dtype=torch.uint8, device=dev)
        b = torch.empty(n, dtype=torch.uint8, device=dev)
        a.fill_(1)
        torch.cuda.synchronize()
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n, "copy_calibration_bytes_written": n}))
        return

    out = {}
    M, K = 8192, 7168
    numel = M * K
    qbytes = wl.quant_bytes(numel)

    # ---- inputs resident in HBM: args.sets independent buffer sets
    xs = [wl.activations_with_outliers(M, K, seed=2026 + i, device=dev) for i in range(args.sets)]
    import hashlib
    input_sha256 = hashlib.sha256(xs[0].view(torch.int16).cpu().numpy().tobytes()).hexdigest()
    qs = [torch.empty((M, K // 2), dtype=torch.uint8, device=dev) for _ in range(args.sets)]
    ss = [torch.empty((M, K // 32), dtype=torch.uint8, device=dev) for _ in range(args.sets)]
    torch.cuda.synchronize()

    def quant(i):
        rc = lib.omo_hip_per_token_group_quant_fp4(xs[i].data_ptr(), numel, qs[i].data_ptr(), numel // 2,
                                                   ss[i].data_ptr(), numel // 32, 32, 1e-10, -6.0, 6.0, 0, cur())
        if rc:
            _abi.check(rc)

    total_ms, eager_ms = time_launches(torch, quant, args.sets, args.steps, args.warmup)
    ms_step = total_ms / args.steps
    # the timed region holds only the quantize launches, so its average
    # launch duration is the region's duration over the launch count
    avg_launch_ms = ms_step
    value = qbytes / (ms_step * 1e-3) / 1e9
    achieved = value
    out["eager_launches"] = {"GB/s": round(qbytes / (eager_ms / args.steps * 1e-3) / 1e9, 1),
                             "us_per_launch": round(eager_ms / args.steps * 1e3, 3),
                             "note": "same launches enqueued one by one from Python instead of one graph replay"}

    # parity of the timed outputs (set 0) against the CPU oracle, and the CPU baseline
    cpu = None
    parity = {}
    oracle = np = None
    nthreads, thread_info = cpu_threads()
    if not args.no_cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import numpy as np
        import oracle
        xb = xs[0].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
        (eq, es), med, reps, spent = cpu_time(lambda: oracle.quant_mxfp4(xb, nthreads=nthreads), args.cpu_seconds)
        parity["quant_cfg2"] = bool(np.array_equal(qs[0].cpu().numpy().reshape(-1), eq) and
                                    np.array_equal(ss[0].cpu().numpy().reshape(-1), es))
        cpu = {"value": round(qbytes / med / 1e9, 3), "unit": "GB/s", "cores": nthreads, "kind": "port",
               "sample": f"oracle quantize of the full 8192x7168 cfg2 tensor on {nthreads} threads, {reps} reps, "
                         f"median {med * 1e3:.1f} ms ({spent:.1f} s of CPU work)",
               "cpu_model": cpu_model(), **thread_info, "per_config": {}}

    def cpu_leg(name, fn, nbytes, check=None, seconds=None):
        """Times the oracle on one more configuration (bounded CPU time) and
        checks the GPU outputs against its result."""
        if cpu is None:
            return
        res, med, reps, spent = cpu_time(fn, seconds or max(1.0, args.cpu_seconds / 4))
        cpu["per_config"][name] = {"GB/s": round(nbytes / med / 1e9, 3), "median_ms": round(med * 1e3, 2),
                                   "reps": reps, "cpu_s": round(spent, 1)}
        if check is not None:
            parity[name] = bool(check(res))

    traffic, traffic_source = None, None
    tpath = os.path.join(ROOT, "profiles", "traffic_quant_phased_cfg2.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            tj = json.load(f)
        traffic = tj.get("hbm_bytes_per_launch")
        import hashlib
        srcs = tj.get("sources_sha256") or {}
        current = {f: hashlib.sha256(open(os.path.join(ROOT, f), "rb").read()).hexdigest()
                   for f in srcs if os.path.exists(os.path.join(ROOT, f))}
        traffic_source = {"file": "profiles/traffic_quant_phased_cfg2.json",
                          "measured_at_commit": tj.get("measured_at_commit"),
                          "method": "median TCC read/write request bytes per dispatch (rocprofv3 --pmc)",
                          "kernel_sources_unchanged": bool(srcs) and current == srcs}

    # ---- extra legs -------------------------------------------------------
    if want("dequant"):
        ys = [torch.empty((M, K), dtype=torch.bfloat16, device=dev) for _ in range(args.sets)]

        def dequant(i):
            rc = lib.omo_hip_per_token_Mxfp4ToBf16_dequant(qs[i].data_ptr(), numel // 2, ss[i].data_ptr(),
                                                           numel // 32, ys[i].data_ptr(), numel, None, 0, 32,
                                                           1e-10, -6.0, 6.0, 0, cur())
            if rc:
                _abi.check(rc)
        steps = max(100, args.steps // 4)
        t, _ = time_launches(torch, dequant, args.sets, steps, 20)
        dq = wl.dequant_bytes(numel)
        out["dequant"] = {"workload": "MXFP4->BF16 8192x7168", "GB/s": round(dq / (t / steps * 1e-3) / 1e9, 1),
                          "us_per_launch": round(t / steps * 1e3, 2),
                          "frac_of_peak": round(dq / (t / steps * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}
        if cpu is not None:
            y0 = ys[0].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
            cpu_leg("dequant_cfg2", lambda: oracle.dequant_bf16(eq, es, nthreads=nthreads), dq,
                    check=lambda r: np.array_equal(r, y0))
        del ys

    if want("cfg1"):
        # cfg1: quantize + dequantize round trip of the seeded 4096 x 4096 N(0,1) tensor
        M1, K1 = wl.CFG1_SHAPE
        n1 = M1 * K1
        b1 = wl.quant_bytes(n1) + wl.dequant_bytes(n1)
        c1s = sets_for(b1, args.sets)
        x1 = [wl.cfg1_input(device=dev)] + [wl.normal_bf16((M1, K1), seed=wl.CFG1_SEED + i, device=dev)
                                             for i in range(1, c1s)]
        q1 = [torch.empty((M1, K1 // 2), dtype=torch.uint8, device=dev) for _ in range(c1s)]
        s1 = [torch.empty((M1, K1 // 32), dtype=torch.uint8, device=dev) for _ in range(c1s)]
        y1 = [torch.empty((M1, K1), dtype=torch.bfloat16, device=dev) for _ in range(c1s)]

        def round_trip(i):
            _abi.check(lib.omo_hip_per_token_group_quant_fp4(x1[i].data_ptr(), n1, q1[i].data_ptr(), n1 // 2,
                                                             s1[i].data_ptr(), n1 // 32, 32, 1e-10, -6.0, 6.0, 0,
                                                             cur()))
            _abi.check(lib.omo_hip_per_token_Mxfp4ToBf16_dequant(q1[i].data_ptr(), n1 // 2, s1[i].data_ptr(),
                                                                 n1 // 32, y1[i].data_ptr(), n1, None, 0, 32, 1e-10,
                                                                 -6.0, 6.0, 0, cur()))
        steps = max(100, args.steps // 4)
        t, _ = time_launches(torch, round_trip, c1s, steps, 20)
        out["cfg1_round_trip"] = {"workload": "cfg1 quantize + dequantize round trip, 4096x4096 N(0,1) bf16",
                                  "GB/s": round(b1 / (t / steps * 1e-3) / 1e9, 1),
                                  "us_per_round_trip": round(t / steps * 1e3, 2),
                                  "algorithmic_bytes": b1}
        if cpu is not None:
            xb1 = x1[0].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
            got = (q1[0].cpu().numpy().reshape(-1), s1[0].cpu().numpy().reshape(-1),
                   y1[0].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1))

            def cpu_round_trip():
                cq_, cs_ = oracle.quant_mxfp4(xb1, nthreads=nthreads)
                return cq_, cs_, oracle.dequant_bf16(cq_, cs_, nthreads=nthreads)
            cpu_leg("cfg1_round_trip", cpu_round_trip, b1,
                    check=lambda r: all(np.array_equal(a, b) for a, b in zip(r, got)))
        del x1, q1, s1, y1

    if want("payload"):
        # cfg4: one GPU's share of the MoE dispatch payload, requant to FP8 and dequant to bf16
        Mp = 4096
        n4 = Mp * K
        ps = sets_for(wl.requant_fp8_bytes(n4), args.sets)
        x4 = wl.normal_bf16((Mp, K), seed=44, device=dev)
        q4 = [torch.empty((Mp, K // 2), dtype=torch.uint8, device=dev) for _ in range(ps)]
        s4 = [torch.empty((Mp, K // 32), dtype=torch.uint8, device=dev) for _ in range(ps)]
        for i in range(ps):
            omo.omo_per_token_group_quant_fp4(x4, q4[i], s4[i], 32, 1e-10, -6.0, 6.0, False)
        f8 = [torch.empty((Mp, K), dtype=torch.float8_e4m3fn, device=dev) for _ in range(ps)]
        f8s = [torch.empty((K // 128, Mp), dtype=torch.float32, device=dev) for _ in range(ps)]

        def requant(i):
            rc = lib.omo_hip_per_token_Mxfp4ToFp8(q4[i].data_ptr(), Mp, K // 2, s4[i].data_ptr(), n4 // 32,
                                                  f8[i].data_ptr(), n4, f8s[i].data_ptr(), n4 // 128, 128, 1e-10,
                                                  -6.0, 6.0, 0, cur())
            if rc:
                _abi.check(rc)
        steps = max(100, args.steps // 4)
        t, _ = time_launches(torch, requant, ps, steps, 20)
        rb = wl.requant_fp8_bytes(n4)
        out["payload_requant_fp8"] = {"workload": "MXFP4->FP8 E4M3 1x128 4096x7168",
                                      "kernel_GB/s": round(rb / (t / steps * 1e-3) / 1e9, 1),
                                      "us_per_launch": round(t / steps * 1e3, 2)}
        y4 = [torch.empty((Mp, K), dtype=torch.bfloat16, device=dev) for _ in range(ps)]

        def deq4(i):
            rc = lib.omo_hip_per_token_Mxfp4ToBf16_dequant(q4[i].data_ptr(), n4 // 2, s4[i].data_ptr(), n4 // 32,
                                                           y4[i].data_ptr(), n4, None, 0, 32, 1e-10, -6.0, 6.0, 0,
                                                           cur())
            if rc:
                _abi.check(rc)
        t, _ = time_launches(torch, deq4, ps, steps, 20)
        db = wl.dequant_bytes(n4)
        out["payload_dequant_bf16"] = {"workload": "MXFP4->BF16 4096x7168",
                                       "kernel_GB/s": round(db / (t / steps * 1e-3) / 1e9, 1),
                                       "us_per_launch": round(t / steps * 1e3, 2)}
        if cpu is not None:
            qn, sn = q4[0].cpu().numpy(), s4[0].cpu().numpy()
            f8g = (f8[0].cpu().view(torch.uint8).numpy(), f8s[0].cpu().numpy())
            y4g = y4[0].cpu().view(torch.int16).numpy().view(np.uint16).reshape(-1)
            cpu_leg("cfg4_requant_fp8", lambda: oracle.mxfp4_to_fp8(qn, sn, nthreads=nthreads), rb,
                    check=lambda r: np.array_equal(r[0], f8g[0]) and np.array_equal(r[1].view(np.uint32),
                                                                                     f8g[1].view(np.uint32)))
            cpu_leg("cfg4_dequant_bf16", lambda: oracle.dequant_bf16(qn, sn, nthreads=nthreads), db,
                    check=lambda r: np.array_equal(r, y4g))
        # transposed FP8 requant (fp8 [2W, M] + fp32 [M/128, 2W]) of the same payload
        fc = [torch.empty((K, Mp), dtype=torch.float8_e4m3fn, device=dev) for _ in range(ps)]
        fcs = [torch.empty((Mp // 128, K), dtype=torch.float32, device=dev) for _ in range(ps)]

        def requant_col(i):
            rc = lib.omo_hip_per_token_Mxfp4ToFp8_col(q4[i].data_ptr(), Mp, K // 2, s4[i].data_ptr(), n4 // 32,
                                                      fc[i].data_ptr(), n4, fcs[i].data_ptr(), n4 // 128, 128,
                                                      1e-10, -6.0, 6.0, 0, cur())
            if rc:
                _abi.check(rc)
        t, _ = time_launches(torch, requant_col, ps, steps, 20)
        out["payload_requant_fp8_col"] = {"workload": "MXFP4->FP8 E4M3 transposed 128x128 tiles 4096x7168",
                                          "kernel_GB/s": round(rb / (t / steps * 1e-3) / 1e9, 1),
                                          "us_per_launch": round(t / steps * 1e3, 2)}
        del q4, s4, f8, f8s, y4, x4, fc, fcs

    if want("ep_payload"):
        # expert-parallel payload rows [codes | scales] at cfg4's share (4096 x 7168): the fused
        # kernels against Megatron's composition (quantize + torch.cat; two .contiguous() split
        # copies + requant / dequant), all enqueued eagerly (torch's cat/copies allocate).
        from omo_python_api import ep_payload as ep
        from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
        from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_wrapper
        Tp, Hp = 4096, K
        n5 = Tp * Hp
        es = sets_for(wl.quant_bytes(n5) + wl.requant_fp8_bytes(n5), args.sets)
        xe = [wl.normal_bf16((Tp, Hp), seed=60 + i, device=dev) for i in range(es)]
        pe = [ep.fp4_quantize_packed(x) for x in xe]
        steps = max(100, args.steps // 4)
        res = {}
        for name, fn in [
            ("send_fused", lambda i: ep.fp4_quantize_packed(xe[i])),
            ("send_unfused", lambda i: ep.join_payload(*omo_per_token_group_quant_mxfp4(xe[i]))),
            ("recv_fp8_fused", lambda i: ep.packed_mxfp4ToFp8(pe[i])),
            ("recv_fp8_unfused", lambda i: omo_per_token_mxfp4ToFp8_wrapper(*ep.split_payload(pe[i]),
                                                                             [Tp])),
            ("recv_bf16_fused", lambda i: ep.packed_mxfp4ToBf16(pe[i])),
        ]:
            t, _ = time_launches(torch, fn, es, steps, 10, graph=False)
            res[name] = round(t / steps * 1e3, 2)
        out["ep_payload"] = {
            "workload": "expert-parallel payload rows [T, 17H/32], T=4096, H=7168 (eager launches, us per call)",
            "us": res,
            "send_speedup": round(res["send_unfused"] / res["send_fused"], 3),
            "recv_fp8_speedup": round(res["recv_fp8_unfused"] / res["recv_fp8_fused"], 3),
            "send_fused_GB/s": round(wl.quant_bytes(n5) / (res["send_fused"] * 1e-6) / 1e9, 1),
            "recv_fp8_fused_GB/s": round(wl.requant_fp8_bytes(n5) / (res["recv_fp8_fused"] * 1e-6) / 1e9, 1),
        }
        del xe, pe

    if want("moe"):
        # cfg5: one MoE layer's MXFP4 codec work on the GPU that owns experts 0-7 of 64
        # (16384 tokens, top-8 of 64, seeded): per-expert rows m_e (ragged, ~2048 each),
        # concatenated [R = sum m_e] where rows are independent.
        c5 = wl.CFG5
        m_e = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["local_experts"]), seed=5)
        R, Hd, Fd = sum(m_e), c5["hidden"], c5["ffn"]
        rows_t = [(R, Hd), (R, Fd), (R, Hd), (R, 2 * Fd)]  # fwd act, fc2 input, bwd grads (fc2, fc1)
        xq = [wl.normal_bf16(sh, seed=70 + i, device=dev) for i, sh in enumerate(rows_t)]
        oq = [(torch.empty((r, c // 2), dtype=torch.uint8, device=dev), torch.empty((r, c // 32), dtype=torch.uint8,
                                                                                   device=dev)) for r, c in rows_t]
        w_shapes = [(Hd, Fd), (Hd, Fd), (Fd, Hd)] * c5["local_experts"]  # gate, up, down per expert
        ws = [wl.normal_bf16(sh, seed=100 + i, device=dev, std=0.02) for i, sh in enumerate(w_shapes)]
        wo = [tuple(torch.empty(shp, dtype=torch.uint8, device=dev)
                    for shp in ((r, c // 2), (r, c // 32), (c, r // 2), (c, r // 32))) for r, c in w_shapes]
        w_items = (_abi.DualItem * len(ws))(*[
            _abi.DualItem(w.data_ptr(), w.size(0), w.size(1), rq_.data_ptr(), rq_.numel(), rs_.data_ptr(), rs_.numel(),
                          cq_.data_ptr(), cq_.numel(), cs_.data_ptr(), cs_.numel()) for w, (rq_, rs_, cq_, cs_) in zip(ws, wo)])
        # wgrad: per-split row -> col FP8 of the activation codes
        lens5, offs5, soffs5, mx5 = (torch.tensor(v, dtype=torch.int32, device=dev) if i < 3 else v
                                     for i, v in enumerate(_split_meta(m_e)))
        srows5 = sum(-(-m // 128) for m in m_e)
        rc_out = torch.empty((R * Hd,), dtype=torch.uint8, device=dev)
        rc_s = torch.empty((srows5, Hd), dtype=torch.float32, device=dev)

        def moe_step(_i):
            for (x, (q, s)) in zip(xq, oq):
                n_ = x.numel()
                _abi.check(lib.omo_hip_per_token_group_quant_fp4(x.data_ptr(), n_, q.data_ptr(), n_ // 2, s.data_ptr(),
                                                                 n_ // 32, 32, 1e-10, -6.0, 6.0, 0, cur()))
            # the 24 expert weights in one grouped launch
            _abi.check(lib.omo_hip_quant_mxfp4_dual_grouped(w_items, len(ws), 1e-10, cur()))
            q0, s0 = oq[0]
            _abi.check(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(
                q0.data_ptr(), R, Hd // 2, s0.data_ptr(), s0.numel(), rc_out.data_ptr(), rc_out.numel(),
                rc_s.data_ptr(), rc_s.numel(), lens5.data_ptr(), offs5.data_ptr(), soffs5.data_ptr(), len(m_e), mx5,
                1e-10, cur()))

        moe_bytes = (sum(wl.quant_bytes(r * c) for r, c in rows_t) + sum(wl.dual_quant_bytes(r * c) for r, c in w_shapes)
                     + sum(wl.row_to_col_fp8_bytes(m, Hd) for m in m_e))
        steps = max(10, args.steps // 50)
        t, _ = time_launches(torch, moe_step, 1, steps, 2)
        out["moe_cfg5"] = {
            "workload": f"cfg5 MoE layer on experts 0-7 of 64: 16384 tokens top-8, R={R} local rows "
                        f"(m_e {min(m_e)}..{max(m_e)}); 4 activation/grad quantizes, 24 weight dual quantizes "
                        "(one grouped launch), per-split row->col FP8",
            "launches_per_step": len(rows_t) + 1 + 1,
            "algorithmic_bytes_per_step": moe_bytes,
            "us_per_step": round(t / steps * 1e3, 1),
            "GB/s": round(moe_bytes / (t / steps * 1e-3) / 1e9, 1),
        }
        del xq, oq, ws, wo, rc_out, rc_s

    if want("dual"):
        Mw, Kw = 7168, 18432
        nw = Mw * Kw
        sets = 2  # 2 x 404 MB exceeds the 256 MB cache
        xw = [wl.heavy_tail_weights(Mw, Kw, seed=33 + i, device=dev) for i in range(sets)]
        rq = [torch.empty((Mw, Kw // 2), dtype=torch.uint8, device=dev) for _ in range(sets)]
        rs = [torch.empty((Mw, Kw // 32), dtype=torch.uint8, device=dev) for _ in range(sets)]
        cq = [torch.empty((Kw, Mw // 2), dtype=torch.uint8, device=dev) for _ in range(sets)]
        cs = [torch.empty((Kw, Mw // 32), dtype=torch.uint8, device=dev) for _ in range(sets)]

        def dual(i):
            rc = lib.omo_hip_quant_mxfp4_dual(xw[i].data_ptr(), Mw, Kw, rq[i].data_ptr(), nw // 2, rs[i].data_ptr(),
                                              nw // 32, cq[i].data_ptr(), nw // 2, cs[i].data_ptr(), nw // 32, 1e-10,
                                              cur())
            if rc:
                _abi.check(rc)
        steps = max(50, args.steps // 10)
        t, _ = time_launches(torch, dual, sets, steps, 10)
        b = wl.dual_quant_bytes(nw)
        out["dual_quant"] = {"workload": "rowwise+columnwise MXFP4 7168x18432",
                             "kernel_GB/s": round(b / (t / steps * 1e-3) / 1e9, 1),
                             "us_per_launch": round(t / steps * 1e3, 2)}
        del xw, rq, rs, cq, cs

    if want("rowcol"):
        Mr, Nr = 4096, 7168
        rs_ = sets_for(wl.row_to_col_fp8_bytes(Mr, Nr), args.sets)
        q5 = [torch.empty((Mr, Nr // 2), dtype=torch.uint8, device=dev) for _ in range(rs_)]
        s5 = [torch.empty((Mr, Nr // 32), dtype=torch.uint8, device=dev) for _ in range(rs_)]
        x5 = wl.normal_bf16((Mr, Nr), seed=55, device=dev)
        for i in range(rs_):
            omo.omo_per_token_group_quant_fp4(x5, q5[i], s5[i], 32, 1e-10, -6.0, 6.0, False)
        o5 = [torch.empty((Nr, Mr), dtype=torch.float8_e4m3fn, device=dev) for _ in range(rs_)]
        os5 = [torch.empty((Mr // 128, Nr), dtype=torch.float32, device=dev) for _ in range(rs_)]

        def rowcol(i):
            rc = lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(q5[i].data_ptr(), Mr, Nr // 2, s5[i].data_ptr(), Mr,
                                                              Nr // 32, o5[i].data_ptr(), Nr, Mr, os5[i].data_ptr(),
                                                              Mr // 128, Nr, 1e-10, cur())
            if rc:
                _abi.check(rc)
        steps = max(100, args.steps // 4)
        t, _ = time_launches(torch, rowcol, rs_, steps, 20)
        b = wl.row_to_col_fp8_bytes(Mr, Nr)
        out["row_to_col_fp8"] = {"workload": "MXFP4 rowwise -> FP8 columnwise 4096x7168",
                                 "kernel_GB/s": round(b / (t / steps * 1e-3) / 1e9, 1),
                                 "us_per_launch": round(t / steps * 1e3, 2)}
        del q5, s5, o5, os5

    if want("rowcol_partial"):
        # a width that is a multiple of 32 but not of 256 (the 256-column tiles' last band
        # partial): dense 4096 x 7040, and cfg5's routed rows x 7040 in their 8 splits
        Mr, Nr = 4096, 7040
        rs_ = sets_for(wl.row_to_col_fp8_bytes(Mr, Nr), args.sets)
        xq = wl.normal_bf16((Mr, Nr), seed=56, device=dev)
        qd = [torch.empty((Mr, Nr // 2), dtype=torch.uint8, device=dev) for _ in range(rs_)]
        sd = [torch.empty((Mr, Nr // 32), dtype=torch.uint8, device=dev) for _ in range(rs_)]
        for i in range(rs_):
            omo.omo_per_token_group_quant_fp4(xq, qd[i], sd[i], 32, 1e-10, -6.0, 6.0, False)
        del xq
        od = [torch.empty((Nr, Mr), dtype=torch.float8_e4m3fn, device=dev) for _ in range(rs_)]
        osd = [torch.empty((Mr // 128, Nr), dtype=torch.float32, device=dev) for _ in range(rs_)]

        def rowcol_p(i):
            _abi.check(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col(
                qd[i].data_ptr(), Mr, Nr // 2, sd[i].data_ptr(), Mr, Nr // 32, od[i].data_ptr(), Nr, Mr,
                osd[i].data_ptr(), Mr // 128, Nr, 1e-10, cur()))
        steps = max(100, args.steps // 4)
        t, _ = time_launches(torch, rowcol_p, rs_, steps, 20)
        b = wl.row_to_col_fp8_bytes(Mr, Nr)
        res = {"dense_workload": "MXFP4 rowwise -> FP8 columnwise 4096x7040",
               "dense_kernel_GB/s": round(b / (t / steps * 1e-3) / 1e9, 1),
               "dense_us_per_launch": round(t / steps * 1e3, 2)}
        del qd, sd, od, osd
        c5 = wl.CFG5
        m_e = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["local_experts"]), seed=5)
        R = sum(m_e)
        b = sum(wl.row_to_col_fp8_bytes(m, Nr) for m in m_e)
        ms_sets = sets_for(b, 3)
        lens7, offs7, soffs7, mx7 = (torch.tensor(v, dtype=torch.int32, device=dev) if i < 3 else v
                                     for i, v in enumerate(_split_meta(m_e)))
        srows7 = sum(-(-m // 128) for m in m_e)
        xq = wl.normal_bf16((R, Nr), seed=71, device=dev)
        q7 = [torch.empty((R, Nr // 2), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        s7 = [torch.empty((R, Nr // 32), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        for i in range(ms_sets):
            omo.omo_per_token_group_quant_fp4(xq, q7[i], s7[i], 32, 1e-10, -6.0, 6.0, False)
        del xq
        o7 = [torch.empty((R * Nr,), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        os7 = [torch.empty((srows7, Nr), dtype=torch.float32, device=dev) for _ in range(ms_sets)]

        def msplit_p(i):
            _abi.check(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(
                q7[i].data_ptr(), R, Nr // 2, s7[i].data_ptr(), s7[i].numel(), o7[i].data_ptr(), o7[i].numel(),
                os7[i].data_ptr(), os7[i].numel(), lens7.data_ptr(), offs7.data_ptr(), soffs7.data_ptr(), len(m_e),
                mx7, 1e-10, cur()))
        steps = max(50, args.steps // 10)
        t, _ = time_launches(torch, msplit_p, ms_sets, steps, 10)
        res.update({"msplit_workload": f"per-split, cfg5's {R} routed rows x {Nr} in {len(m_e)} splits",
                    "msplit_kernel_GB/s": round(b / (t / steps * 1e-3) / 1e9, 1),
                    "msplit_us_per_launch": round(t / steps * 1e3, 2)})
        out["row_to_col_partial_band"] = res
        del q7, s7, o7, os7

    if want("msplit"):
        # cfg5's per-split row -> col FP8 alone (the moe leg runs it after the grouped weight
        # quantize, whose written lines it inherits): the 16431 routed rows of experts 0-7 in
        # their 8 ragged splits, rotating buffer sets.
        c5 = wl.CFG5
        m_e = wl.moe_routing(c5["tokens"], c5["n_experts"], c5["topk"], range(c5["local_experts"]), seed=5)
        R, Hd = sum(m_e), c5["hidden"]
        b = sum(wl.row_to_col_fp8_bytes(m, Hd) for m in m_e)
        ms_sets = sets_for(b, 3)
        lens6, offs6, soffs6, mx6 = (torch.tensor(v, dtype=torch.int32, device=dev) if i < 3 else v
                                     for i, v in enumerate(_split_meta(m_e)))
        srows6 = sum(-(-m // 128) for m in m_e)
        x6 = wl.normal_bf16((R, Hd), seed=70, device=dev)
        q6 = [torch.empty((R, Hd // 2), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        s6 = [torch.empty((R, Hd // 32), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        for i in range(ms_sets):
            omo.omo_per_token_group_quant_fp4(x6, q6[i], s6[i], 32, 1e-10, -6.0, 6.0, False)
        del x6
        o6 = [torch.empty((R * Hd,), dtype=torch.uint8, device=dev) for _ in range(ms_sets)]
        os6 = [torch.empty((srows6, Hd), dtype=torch.float32, device=dev) for _ in range(ms_sets)]

        def msplit(i):
            _abi.check(lib.omo_hip_per_token_Mxfp4RowToBf16ToFp8Col_msplit(
                q6[i].data_ptr(), R, Hd // 2, s6[i].data_ptr(), s6[i].numel(), o6[i].data_ptr(), o6[i].numel(),
                os6[i].data_ptr(), os6[i].numel(), lens6.data_ptr(), offs6.data_ptr(), soffs6.data_ptr(), len(m_e),
                mx6, 1e-10, cur()))
        steps = max(50, args.steps // 10)
        t, _ = time_launches(torch, msplit, ms_sets, steps, 10)
        out["msplit_cfg5"] = {"workload": f"per-split MXFP4 row -> FP8 col alone, cfg5's {R} routed rows x {Hd} in "
                                          f"{len(m_e)} splits ({min(m_e)}..{max(m_e)} rows)",
                              "kernel_GB/s": round(b / (t / steps * 1e-3) / 1e9, 1),
                              "us_per_launch": round(t / steps * 1e3, 2)}
        del q6, s6, o6, os6

    if want("permute"):
        # TE's moe_permute on an MXFP4 tensor at one rank's share: 4096 tokens routed top-8 of 64
        # experts (seeded), H = 7168, 32768 expert-major output rows. The row map is built once
        # (make_row_id_map synchronizes with the host); timed are the gather, the gather fused
        # into the FP8 requant, and the gather followed by the requant (eager launches).
        import omo
        from omo_python_api import permutation as pm
        from omo_python_api.mxfp4 import omo_per_token_group_quant_mxfp4
        from omo_python_api.mxfp4_dequant import omo_per_token_mxfp4ToFp8_wrapper
        Tq, Hq, Eq, topk = 4096, K, 64, 8
        gq = torch.Generator(device="cpu").manual_seed(81)
        rmap = torch.zeros((Tq, Eq), dtype=torch.bool)
        rmap.scatter_(1, torch.rand((Tq, Eq), generator=gq).topk(topk, dim=1).indices, True)
        cq, csq = omo_per_token_group_quant_mxfp4(wl.normal_bf16((Tq, Hq), seed=82, device=dev))
        src, _, _ = pm.make_row_id_map(rmap.to(dev))
        Np = src.numel()
        gq_out = (torch.empty((Np, Hq // 2), dtype=torch.uint8, device=dev),
                  torch.empty((Np, Hq // 32), dtype=torch.uint8, device=dev))
        fq_out = (torch.empty((Np, Hq), dtype=torch.float8_e4m3fn, device=dev),
                  torch.empty((Hq // 128, Np), dtype=torch.float32, device=dev))

        def unfused(_i):
            omo.omo_mxfp4_permute_rows(cq, csq, src, *gq_out)
            return omo_per_token_mxfp4ToFp8_wrapper(*gq_out, [Np])

        row_b, fp8_b = Hq // 2 + Hq // 32, Hq + Hq // 128 * 4
        steps = max(100, args.steps // 4)
        res = {}
        for name, fn in [("gather", lambda i: omo.omo_mxfp4_permute_rows(cq, csq, src, *gq_out)),
                         ("gather_to_fp8_fused", lambda i: omo.omo_permute_Mxfp4ToFp8(cq, csq, src, *fq_out)),
                         ("gather_then_fp8", unfused)]:
            t, _ = time_launches(torch, fn, 1, steps, 10, graph=False)
            res[name] = round(t / steps * 1e3, 2)
        out["permute"] = {
            "workload": f"MXFP4 moe_permute, {Tq} tokens top-{topk} of {Eq} experts -> {Np} rows, H={Hq} "
                        "(eager launches, us per call)",
            "us": res,
            "fused_speedup": round(res["gather_then_fp8"] / res["gather_to_fp8_fused"], 3),
            "gather_GB/s": round(2 * Np * row_b / (res["gather"] * 1e-6) / 1e9, 1),
            "gather_to_fp8_fused_GB/s": round(Np * (row_b + fp8_b) / (res["gather_to_fp8_fused"] * 1e-6) / 1e9, 1),
            "bytes": "rows moved: gather 2 x rows x (H/2 + H/32); fused rows x (H/2 + H/32 + H + 4H/128)",
        }
        del cq, csq, gq_out, fq_out

    if want("ceiling"):
        try:
            out["memory_ceiling"] = ceiling_leg(torch, args, dev, cur, xs, qs, ss, numel, qbytes, value)
        except (OSError, RuntimeError) as e:  # an optional leg: report, never lose the bench line
            out["memory_ceiling"] = {"error": str(e)}

    if "floors" in only:
        try:
            out["pattern_floors"] = floors_leg(torch, args, dev, cur, lib, _abi, wl)
        except (OSError, RuntimeError) as e:
            out["pattern_floors"] = {"error": str(e)}

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg2 per-token BF16->MXFP4 quantize, 8192x7168, N(0,1) with 0.1% of channels "
                               "x100, rowwise 1x32 E2M1 + E8M0", "rows": M, "cols": K,
                   "algorithmic_bytes_per_step": qbytes, "buffer_sets": args.sets,
                   "input_sha256": input_sha256},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": traffic_source,
                     "kernel": "quant_phased_kernel", "avg_launch_us": round(avg_launch_ms * 1e3, 3)},
        "cpu_baseline": cpu,
        "parity_vs_oracle": all(parity.values()) if parity else None,
        "parity_detail": parity or None,
        "timing": "eager launches" if args.eager else "one HIP-graph replay of the timed launches",
    }
    line.update(out)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
