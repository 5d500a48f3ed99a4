"""Headline benchmark: exact 10-NN queries/sec over 10M x 128 uint8 vectors (L2) on one MI355X.

    python bench.py [--gpus 1] [--steps 5] [--warmup 1]

A step is one search of all 10,000 queries (k = 10) against the 10,000,000-row index, with the
index built and the queries resident in HBM before the timed region. The data follow config 2:
1,000 centres uniform in [0, 80]^128, each vector a random centre plus N(0, 20^2) per coordinate,
rounded half-to-even and clipped to [0, 255]; drawn with torch generators seeded 1 (centres), 2
(base) and 3 (queries). The index stores its rows in the order of 4,096 k-means lists (built
with the index; --lists 0 keeps id order) and the searches probe none of them (--probe 0): every
row is screened, and similar consecutive rows switch fewer bits in the MFMA (about 3% faster
screen, measured); the thresholds come from the anchors of each query's 8 nearest lists. Prints one JSON line with the roofline of the dominant kernel (the int8
MFMA screen, timed with HIP events inside the library over the timed steps) and the CPU oracle's
exhaustive fp64 search timed on the first queries against the full base.
"""

import argparse
import ctypes
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

P_INT8_TOPS = 5000.0  # MI355X dense int8 MFMA peak, 10^12 ops/s (256 CUs at 2.4 GHz)
PEAK_CLOCK_MHZ = 2400.0  # the shader clock the datasheet peaks assume
TRAFFIC_PROFILE = os.path.join(ROOT, "profiles", "screen_i8_c2_traffic.txt")
# the sources that decide a screen's memory traffic; a traffic profile is stamped with their hash
# and is used only while they are unchanged
SCREEN_I8_SOURCES = ("kernels/screen.hip", "kernels/screen_common.hpp", "kernels.hpp")
# every kernel source: the stamp of the config 3 and 4 counter profiles
KERNEL_SOURCES = ("kernels/screen.hip", "kernels/screen_tile.hip", "kernels/screen_wide.hip",
                  "kernels/screen_common.hpp", "kernels/select.hip", "kernels/encode.hip",
                  "kernels/partition.hip", "kernels/lists.hip", "kernels.hpp")
PROFILE_C3 = os.path.join(ROOT, "profiles", "screen_f16_c3_counters.txt")
PROFILE_C4 = os.path.join(ROOT, "profiles", "screen_f16_c4_counters.txt")


def sources_stamp(files=SCREEN_I8_SOURCES):
    """First 16 hex digits of the SHA-256 over the given sources (paths under libcertex_amd/csrc)."""
    import hashlib

    h = hashlib.sha256()
    for f in files:
        with open(os.path.join(ROOT, "libcertex_amd", "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def profile_traffic(path=TRAFFIC_PROFILE, kernel=None, files=SCREEN_I8_SOURCES):
    """HBM bytes per launch of a kernel from a committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary
    (calibrated against a plain copy): its line `traffic_bytes_per_launch <kernel> = N` (the first
    such line when kernel is None). None when the summary is missing or was measured on other
    sources than the ones built here (its `sources_stamp` line differs from the stamp of `files`)."""
    stamp, traffic = None, None
    try:
        for line in open(path):
            if line.startswith("sources_stamp"):
                stamp = line.split("=")[1].strip()
            if line.startswith("traffic_bytes_per_launch") and traffic is None:
                name = line.split("=")[0][len("traffic_bytes_per_launch"):].strip()
                if kernel is None or name.startswith(kernel):
                    traffic = int(line.split("=")[1])
    except OSError:
        return None
    return traffic if stamp == sources_stamp(files) else None


def screen_traffic():
    """HBM bytes per int8 screen launch at config 2 (profiles/screen_i8_c2_traffic.txt)."""
    return profile_traffic()


def shader_clock_mhz():
    """Average shader clock (MHz) of the screen workgroups of the last timed region, as the
    kernels read it (s_memtime cycles over s_memrealtime time); None if no screen ran."""
    from libcertex_amd import _capi as C

    mhz = ctypes.c_double(0)
    C.check(C.lib().cuvsCertexTimingShaderClock(ctypes.byref(mhz)))
    return round(mhz.value, 1) if mhz.value > 0 else None


def clock_fields(achieved, peak):
    """The screen's shader clock and its fraction of the peak scaled to that clock (the datasheet
    peak assumes 2.4 GHz): what the line's frac leaves to the clock, and what to the kernel."""
    mhz = shader_clock_mhz()
    if mhz is None:
        return {"shader_clock_mhz": None}
    return {"shader_clock_mhz": mhz,
            "frac_of_peak_at_clock": round(achieved / (peak * mhz / PEAK_CLOCK_MHZ), 4)}
P_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA peak
HBM_GBS = 8000.0


def mixture_u8(n, d, n_centres, centres, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.uint8, device=device)
    step = 1 << 20
    for i in range(0, n, step):
        m = min(step, n - i)
        c = torch.randint(0, n_centres, (m,), generator=g, device=device)
        v = centres[c] + torch.randn((m, d), generator=g, device=device) * 20.0
        out[i : i + m] = v.round().clamp_(0, 255).to(torch.uint8)
    return out


def powerlaw_unit(n, d, seed, basis, device):
    """Config 3 rows: Gaussian with covariance eigenvalues ~ 1 / i in the orthogonal basis, then
    L2-normalised (torch generator seeded `seed`)."""
    g = torch.Generator(device=device).manual_seed(seed)
    out = torch.empty((n, d), dtype=torch.float32, device=device)
    step = 1 << 17
    for i in range(0, n, step):
        m = min(step, n - i)
        x = torch.randn((m, d), generator=g, device=device) @ basis
        out[i : i + m] = x / x.norm(dim=1, keepdim=True)
    return out


def timed_steps(step, steps, warmup):
    """Runs warmup + steps calls of step(); returns (ms per step, kernel ms per phase, launches)."""
    from libcertex_amd import _capi as C

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    L = C.lib()
    C.check(L.cuvsCertexTimingBegin())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (ctypes.c_double * 4)()
    launches = (ctypes.c_int64 * 4)()
    C.check(L.cuvsCertexTimingEnd(ms, launches))
    return (t1 - t0) * 1000.0 / steps, list(ms), list(launches)


PHASES = ("anchors", "threshold", "screen", "verify_topk")
CPU_TARGET_S = 12.0  # CPU work of the baseline's timed sample, about


def cpu_baseline(run, nq, first, what):
    """The oracle timed on the host on a bounded sample: run(c) searches the first c queries and
    returns their ids. `first` queries are timed first; the sample then grows to about CPU_TARGET_S
    seconds of work (at most nq queries) and is timed again, and once more while it took under half
    of that (the first, small sample also pays the start-up, so it overstates the time per query).
    Returns (record, c, ids)."""
    import oracle

    c = min(first, nq)
    t0 = time.perf_counter()
    ids = run(c)
    t = time.perf_counter() - t0
    for _ in range(2):
        if t >= CPU_TARGET_S / 2 or c >= nq:
            break
        c = int(min(nq, max(c + 1, c * CPU_TARGET_S / max(t, 1e-3))))
        t0 = time.perf_counter()
        ids = run(c)
        t = time.perf_counter() - t0
    rec = {"value": round(c / t, 3), "unit": "queries/s", "cores": oracle.threads(), "kind": "port",
           "cpu": oracle.cpu_model(),
           "sample": f"first {c} of the {nq} queries, {what} (oracle/oracle.c type-specialised scorers, "
           f"OpenMP), {t:.1f} s"}
    return rec, c, ids


def hbm_roofline(kernel, bytes_per_launch, ms_per_launch, what):
    """Roofline of an HBM-bound phase: algorithmic bytes per launch (stated in `what`) over the
    launch's average duration (HIP events of the library), against 8 TB/s."""
    gbs = bytes_per_launch / (ms_per_launch / 1000.0) / 1e9 if ms_per_launch > 0 else 0.0
    return {"bound": "hbm", "kernel": kernel, "achieved": round(gbs, 1), "peak": HBM_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_GBS, 4), "bytes_per_launch": int(bytes_per_launch),
            "avg_launch_ms": round(ms_per_launch, 4), "bytes": what}


def float_phase_rooflines(ms, launches, steps, st, nq, d, k, elem, traffic=None):
    """Verify roofline of a float search (one batch per step): the verify reads every survivor's
    bucket entry (row and screen value), the query and the vectors of the rows it scores, `elem`
    bytes per coordinate (the index's vector type: 4 for float32, 2 for bfloat16 or float16)."""
    v_ms = ms[3] / max(1, launches[3])
    per_launch = max(1, launches[3] // steps)
    r = hbm_roofline(
        "verify_topk_f_kernel", (st.verified * d * elem + st.survivors * 8 + nq * d * elem) / per_launch,
        v_ms, f"{st.verified / max(1, st.queries):.1f} scored vectors of {d} x {elem} B and "
        f"{st.survivors / max(1, st.queries):.1f} bucket entries of 8 B, per query")
    r["traffic"] = traffic
    return {"verify_topk": r}


def bench_config3(args):
    """Config 3: exact 100-NN, cosine, 1,000,000 x 768 fp32 power-law embeddings, 10,000 queries,
    one of 16 labels per vector and per query (label-filtered search), fp16 MFMA screen."""
    import libcertex_amd as certex

    dev = torch.device("cuda:0")
    n, d, nq, k = args.n or 1_000_000, args.dim or 768, args.nq, args.k or 100
    qm, _ = torch.linalg.qr(torch.randn((d, d), generator=torch.Generator().manual_seed(31), dtype=torch.float64))
    basis = (torch.sqrt(1.0 / torch.arange(1, d + 1, dtype=torch.float64))[:, None] * qm.T).float().to(dev)
    X = powerlaw_unit(n, d, 32, basis, dev)
    Q = powerlaw_unit(nq, d, 33, basis, dev)
    gl = torch.Generator(device=dev).manual_seed(34)
    lx = torch.randint(0, 16, (n,), generator=gl, device=dev, dtype=torch.int32)
    lq = torch.randint(0, 16, (nq,), generator=gl, device=dev, dtype=torch.int32)
    idx = certex.Index(d, metric="cosine", **({"anchor_stride": args.stride} if args.stride > 0 else {}))
    idx.add(X, labels=lx)
    torch.cuda.synchronize()
    batch = args.batch or 10_000

    def step():
        return idx.search(Q, k=k, batch=batch, labels=lq)

    ms_step, ms, launches = timed_steps(step, args.steps, args.warmup)
    with certex.search_stats() as st:
        D, I = step()
    torch.cuda.synchronize()
    halves = (d + 127) // 128 * 128
    screen_ms = ms[2] / max(1, launches[2])
    elem = idx.dtype.itemsize
    # the committed counter profile holds the default workload's traffic
    default = (n, d, nq, k, batch, idx.anchor_stride) == (1_000_000, 768, 10_000, 100, 10_000, 16)
    # algorithmic work of the label-routed screen: every query against the rows of its label
    per_label = torch.bincount(lx.long(), minlength=16)
    pairs = float(per_label[lq.long()].sum().item())
    flops_per_launch = 2.0 * pairs * halves / max(1, launches[2] // args.steps)
    achieved = flops_per_launch / (screen_ms / 1000.0) / 1e12
    cpu = None
    if not args.no_cpu:
        import numpy as np

        import oracle

        Xh, Qh, lxh, lqh = X.cpu().numpy(), Q.cpu().numpy(), lx.cpu().numpy(), lq.cpu().numpy()
        cpu, cq, i_cpu = cpu_baseline(
            lambda c: oracle.knn(Xh, Qh[:c], k, "cosine", row_labels=lxh, query_labels=lqh[:c])[1], nq,
            args.cpu_queries, f"exhaustive fp64 over all {n} rows with the label filter")
        cpu["sample"] += f"; ids equal to the GPU's: {bool(np.array_equal(i_cpu, I[:cq].cpu().numpy()))}"
    return {
        "metric": "exact 100-NN queries/sec, 1M x 768 fp32 cosine, 16 labels, 1 MI355X",
        "value": round(nq / (ms_step / 1000.0), 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 screen, f64 re-rank",
        "data": "synthetic (config 3 power-law embeddings, torch generators seeded 31/32/33/34)",
        "config": {
            "workload": f"config 3: exact {k}-NN, cosine, base {n} x {d} fp32, {nq} queries, 16 labels",
            "n": n, "dim": d, "n_queries": nq, "k": k, "batch": batch, "anchor_stride": idx.anchor_stride,
            "phase_ms_per_step": {p: round(ms[i] / args.steps, 4) for i, p in enumerate(PHASES)},
            "launches_per_step": {p: launches[i] // args.steps for i, p in enumerate(PHASES)},
            "survivors_per_query": round(st.survivors / max(1, st.queries), 2),
            "verified_per_query": round(st.verified / max(1, st.queries), 2),
            "phase_rooflines": float_phase_rooflines(
                ms, launches, args.steps, st, nq, d, k, elem,
                profile_traffic(PROFILE_C3, "verify_topk_f_kernel", KERNEL_SOURCES) if default else None),
        },
        "roofline": {
            "bound": "mfma", "kernel": "screen_tile_kernel (fp16 MFMA screen, LDS-staged 256-row x 128-query tiles, two workgroups per CU, label-routed)",
            "achieved": round(achieved, 2), "peak": P_FP16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / P_FP16_TFLOPS, 4),
            "traffic": profile_traffic(PROFILE_C3, "screen_tile_kernel", KERNEL_SOURCES) if default else None,
            "avg_launch_ms": round(screen_ms, 4), "flops_per_launch": flops_per_launch,
            **clock_fields(achieved, P_FP16_TFLOPS),
        },
        "cpu_baseline": cpu,
    }


def bench_config4(args):
    """Config 4: sparse-attention exact top-k over a KV cache (KeyCache / topk), inner product,
    bf16: 8 KV heads x 131,072 keys x 128, 32 query heads (GQA 4:1) x 64 decode queries, k = 2048;
    a step appends 256 new keys per KV head, then runs topk for all query heads."""
    import libcertex_amd as certex

    dev = torch.device("cuda:0")
    n_kv, n, d, H, m, k, grow = 8, args.n or 131_072, args.dim or 128, 32, 64, args.k or 2048, 256
    g = torch.Generator(device=dev).manual_seed(41)
    outliers = torch.randperm(d, generator=torch.Generator().manual_seed(42))[:4].to(dev)

    def keys(count):
        x = torch.randn((n_kv, count, d), generator=g, device=dev)
        x[:, :, outliers] *= 20.0
        return x.to(torch.bfloat16)

    cache = certex.KeyCache(n_kv, d, k=k, capacity=n + grow * (args.warmup + args.steps + 2))
    first = keys(n)
    cache.append(first)
    q = torch.randn((H, m, d), generator=g, device=dev).to(torch.bfloat16)
    torch.cuda.synchronize()
    new_keys = [keys(grow) for _ in range(args.warmup + args.steps + 1)]
    used = []

    def step():
        used.append(new_keys[len(used)])
        cache.append(used[-1])
        return cache.topk(q, k)

    ms_step, ms, launches = timed_steps(step, args.steps, args.warmup)
    with certex.search_stats() as st:
        scores, ids = step()
    torch.cuda.synchronize()
    cpu = None
    if not args.no_cpu:
        import numpy as np

        import oracle

        # the keys of KV head 0 as the cache holds them (float32 holds bf16 exactly)
        head0 = torch.cat([kk[0] for kk in [first] + used], 0).float().cpu().numpy()
        q0 = q[0].float().cpu().numpy()
        cpu, cq, i_cpu = cpu_baseline(
            lambda c: oracle.knn(head0, q0[:c], k, "ip")[1], m, args.cpu_queries,
            f"query head 0 against KV head 0 ({head0.shape[0]} keys), exhaustive fp64")
        cpu["sample"] += f"; ids equal to the GPU's: {bool(np.array_equal(i_cpu, ids[0, :cq].cpu().numpy()))}"
    n_q = H * m
    # screen roofline per step: every query against the keys of its KV head (fp16 rows of 128
    # halves); the cache holds n + 256 (warmup + i + 1) keys per head in timed step i
    keys_avg = n + grow * (args.warmup + (args.steps + 1) / 2.0)
    flops_per_step = 2.0 * n_q * keys_avg * ((d + 127) // 128 * 128)
    screen_ms_step = ms[2] / args.steps
    achieved = flops_per_step / (screen_ms_step / 1000.0) / 1e12
    elem = cache.index.dtype.itemsize  # bfloat16 keys: 2 bytes per coordinate
    default = (n, d, k) == (131_072, 128, 2048)
    return {
        "metric": "exact top-2048 attention queries/sec, 8 KV heads x 131k keys, GQA 4:1, 1 MI355X",
        "value": round(n_q / (ms_step / 1000.0), 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 keys (bf16 exact), f16 screen, f64 re-rank",
        "data": "synthetic (config 4: N(0,1) bf16 keys with 4 channels x20, torch generators seeded 41/42)",
        "config": {
            "workload": f"config 4: {n_kv} KV heads x {n} keys x {d}, {H} query heads x {m} queries, k = {k}, "
            f"+{grow} keys per head per step",
            "phase_ms_per_step": {p: round(ms[i] / args.steps, 4) for i, p in enumerate(PHASES)},
            "launches_per_step": {p: launches[i] // args.steps for i, p in enumerate(PHASES)},
            "survivors_per_query": round(st.survivors / max(1, st.queries), 2),
            "verified_per_query": round(st.verified / max(1, st.queries), 2),
            "phase_rooflines": float_phase_rooflines(
                ms, launches, args.steps, st, n_q, d, k, elem,
                profile_traffic(PROFILE_C4, "verify_topk_f_kernel", KERNEL_SOURCES) if default else None),
        },
        "roofline": {
            "bound": "mfma", "kernel": "screen_kernel<f16_rows,4,...> (fp16 MFMA screen, label-routed, + tail)",
            "achieved": round(achieved, 2), "peak": P_FP16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / P_FP16_TFLOPS, 4),
            "traffic": profile_traffic(PROFILE_C4, "screen_kernel<f16_rows", KERNEL_SOURCES) if default else None,
            "screen_ms_per_step": round(screen_ms_step, 4), "flops_per_step": flops_per_step,
            **clock_fields(achieved, P_FP16_TFLOPS),
        },
        "cpu_baseline": cpu,
    }


def bench_config5(args):
    """Config 5: exact 10-NN, L2, 1,000,000,000 x 128 uint8 (the config 2 mixture, 128 GB of codes
    resident in HBM), 10,000 queries; while the timed searches run, another thread extends the
    index by 1,000,000 rows and removes 1,000,000 random ids. Afterwards 16 queries are checked
    against a GPU fp64 brute force over the live set (exact for 8-bit data). The config's 4,096
    k-means lists (a speed option: the rows stored in list order, the anchors of each query's 8
    nearest lists bounding its threshold; --probe 2 probes the 2 nearest lists' rows instead) need
    the whole base in one build: it is generated into host memory (128 GB) and built
    from there; --lists 0 builds by chunks without lists instead."""
    import threading

    import libcertex_amd as certex

    dev = torch.device("cuda:0")
    n, d, nq, k = args.n or 1_000_000_000, 128, args.nq, args.k or 10
    n_new, n_gone, chunk = 1_000_000, 1_000_000, 10_000_000
    centres = torch.rand((1000, d), generator=torch.Generator().manual_seed(1), dtype=torch.float64) * 80.0
    centres = centres.float().to(dev)

    def rows(i, m):  # chunk i of the base, regenerated on demand (seed 100 + i); the new rows: i = -1
        return mixture_u8(m, d, 1000, centres, 100 + i if i >= 0 else 99, dev)

    n_lists = 4096 if args.lists < 0 else args.lists
    args.probe = 0 if args.probe < 0 else args.probe
    idx = certex.Index(d, metric="l2", capacity=n + n_new, n_lists=n_lists)
    t_build = time.perf_counter()
    if n_lists > 0:
        X = torch.empty((n, d), dtype=torch.uint8)  # host memory: the base for one build
        for c in range(0, n, chunk):
            X[c : c + min(chunk, n - c)] = rows(c // chunk, min(chunk, n - c)).cpu()
            if (c // chunk) % 10 == 9:
                print(f"# generated {c + chunk} rows", file=sys.stderr, flush=True)
        t_build = time.perf_counter()
        idx.add(X)
        del X
    else:
        for c in range(0, n, chunk):
            idx.add(rows(c // chunk, min(chunk, n - c)))
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build
    print(f"# built {n} rows with {n_lists} lists in {t_build:.1f} s", file=sys.stderr, flush=True)
    Q = mixture_u8(nq, d, 1000, centres, 3, dev)
    new = rows(-1, n_new)
    gone = torch.randint(0, n, (n_gone,), generator=torch.Generator(device=dev).manual_seed(4), device=dev)
    torch.cuda.synchronize()
    batch = args.batch or 10_000

    def step():
        return idx.search(Q, k=k, batch=batch, probe_lists=args.probe)

    errors = []

    def writer():
        try:
            with torch.cuda.stream(torch.cuda.Stream()):
                idx.add(new)
                idx.remove(gone)
                torch.cuda.current_stream().synchronize()
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    w = threading.Thread(target=writer)
    w.start()
    ms_step, ms, launches = timed_steps(step, args.steps, 0)
    w.join()
    if errors:
        raise errors[0]
    D, I = step()
    torch.cuda.synchronize()

    # 16 queries against a GPU fp64 brute force over the live set (distances are integers below
    # 2^23 and ids below 2^30: distance * 2^30 + id is an exact total order in fp64)
    live_gone = torch.zeros(n + n_new, dtype=torch.bool, device=dev)
    live_gone[gone] = True
    Qd = Q[:16].double()
    qq = (Qd * Qd).sum(1, keepdim=True)
    best = torch.empty((16, 0), dtype=torch.float64, device=dev)
    for c in range(0, n + n_new, chunk):
        m = min(chunk, n - c) if c < n else n_new
        X = rows(c // chunk, m) if c < n else new
        for s0 in range(0, m, 1_000_000):
            Xc = X[s0 : s0 + 1_000_000].double()
            dist = qq + (Xc * Xc).sum(1)[None] - 2.0 * (Qd @ Xc.T)
            key = dist * float(1 << 30) + torch.arange(c + s0, c + s0 + Xc.shape[0], device=dev, dtype=torch.float64)[None]
            key[:, live_gone[c + s0 : c + s0 + Xc.shape[0]]] = float("inf")
            best = torch.topk(torch.cat([best, key], 1), k, dim=1, largest=False).values
        if c >= n:
            break
    exact_ids = torch.remainder(best, float(1 << 30)).long()
    agree = bool(torch.equal(exact_ids, I[:16]))

    screen_ms = ms[2] / max(1, launches[2])
    batches = (nq + batch - 1) // batch
    ops_per_launch = 2.0 * n * d * nq / batches
    achieved = ops_per_launch / (screen_ms / 1000.0) / 1e12
    return {
        "metric": "exact 10-NN queries/sec, 1B x 128 uint8 L2 with concurrent extend and remove, 1 MI355X",
        "value": round(nq / (ms_step / 1000.0), 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (config 2 mixture per 10M-row chunk, torch generators seeded 1 / 100+i / 99 / 3 / 4)",
        "config": {
            "workload": f"config 5: exact {k}-NN, L2, base {n} x {d} uint8, {nq} queries, +{n_new} rows and "
            f"-{n_gone} random ids during the timed searches",
            "n_lists": n_lists,
            "probe_lists": args.probe if n_lists else 0,
            "build_s": round(t_build, 1),
            "phase_ms_per_step": {p: round(ms[i] / args.steps, 4) for i, p in enumerate(PHASES)},
            "ids_equal_to_brute_force_16_queries": agree,
        },
        "roofline": {
            "bound": "mfma", "kernel": "screen_kernel<int8_rows,2,512,false,false,8,2,false> (int8 MFMA screen, 128-row steps)",
            "achieved": round(achieved, 2), "peak": P_INT8_TOPS, "unit": "TOP/s",
            "frac": round(achieved / P_INT8_TOPS, 4), "traffic": None,
            "avg_launch_ms": round(screen_ms, 4), "ops_per_launch": ops_per_launch,
            **clock_fields(achieved, P_INT8_TOPS),
        },
        "cpu_baseline": None,
    }


def summarize_profiles(dirs, warmup, steps, after=1):
    """Text summary of rocprofv3 CSV output (kernel traces and counter collections) under `dirs`,
    for a bench run of `warmup` + `steps` searches followed by `after` more (the survivor stats).
    A kernel launched L = calls // (warmup + steps + after) >= 1 times per search is averaged over
    all its launches and, separately, over the timed ones only: in dispatch order, the steps * L
    launches before the last after * L (the first search may launch a kernel more often, when its
    survivor buckets grow). Kernels launched fewer times, and the index build's kernels (every
    dispatch before the first of a screen kernel), show '-' there. Durations in ms, counters per
    dispatch."""
    import csv
    import glob
    import re
    from collections import defaultdict

    searches = warmup + steps + after

    def short(name):  # "void ns::(anonymous namespace)::k<ns::T, 2>(args)" -> "k<T, 2>"
        name = re.sub(r"^void ", "", name.strip())
        depth, cut = 0, len(name)
        for i, ch in enumerate(name):  # the first "(" outside template brackets opens the arguments
            depth += ch == "<"
            depth -= ch == ">"
            if ch == "(" and depth == 0 and not name.startswith("(anonymous", i):
                cut = i
                break
        return re.sub(r"(\(anonymous namespace\)::|\b\w+::)", "", name[:cut]).strip()

    def timed(vals):
        per = len(vals) // searches
        if per == 0:
            return None
        sel = vals[len(vals) - (steps + after) * per : len(vals) - after * per]
        return sum(sel) / len(sel) if sel else None

    def data_gen(name):
        return " at::" in name or name.startswith("at::") or name.startswith("Cijk_")

    traces, counters = defaultdict(list), defaultdict(list)
    for d in dirs:
        for f in sorted(glob.glob(os.path.join(d, "**", "*kernel_trace.csv"), recursive=True)):
            for r in csv.DictReader(open(f)):
                if data_gen(r["Kernel_Name"]):
                    continue
                traces[short(r["Kernel_Name"])].append(
                    (int(r["Dispatch_Id"]), (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6))
        for f in sorted(glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True)):
            for r in csv.DictReader(open(f)):
                if data_gen(r["Kernel_Name"]):
                    continue
                counters[(short(r["Kernel_Name"]), r["Counter_Name"])].append(
                    (int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    # the searches start with the first screen launch (the index build's kernels all run before)
    first = {}
    for kind in (traces, counters):
        for key, v in kind.items():
            name = key if isinstance(key, str) else key[0]
            if name.startswith("screen_"):
                first[id(kind)] = min(first.get(id(kind), 1 << 62), min(d for d, _ in v))

    def build_only(kind, v):
        return id(kind) in first and max(d for d, _ in v) < first[id(kind)]

    out = [f"# {searches} searches per run: {warmup} warm-up, {steps} timed, {after} after (stats); "
           "torch's and hipBLASLt's data-generation kernels left out"]
    if traces:
        out.append(f"{'kernel':<64} {'calls':>5} {'total_ms':>10} {'avg_ms':>9} {'timed_avg_ms':>12} "
                   f"{'min_ms':>8} {'max_ms':>8}")
        rows = sorted(traces.items(), key=lambda kv: -sum(v for _, v in kv[1]))
        for name, v in rows:
            v.sort()
            t = [x for _, x in v]
            ta = None if build_only(traces, v) else timed(t)
            out.append(f"{name[:64]:<64} {len(t):>5} {sum(t):>10.3f} {sum(t) / len(t):>9.4f} "
                       f"{(f'{ta:.4f}' if ta is not None else '-'):>12} {min(t):>8.4f} {max(t):>8.4f}")
    if counters:
        out.append(f"{'kernel':<64} {'counter':<28} {'calls':>5} {'avg':>16} {'timed_avg':>16}")
        for (name, cn), v in sorted(counters.items()):
            v.sort()
            t = [x for _, x in v]
            ta = None if build_only(counters, v) else timed(t)
            out.append(f"{name[:64]:<64} {cn:<28} {len(t):>5} {sum(t) / len(t):>16.1f} "
                       f"{(f'{ta:.1f}' if ta is not None else '-'):>16}")
    return "\n".join(out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5),
                    help="2: the headline (10M x 128 uint8); 3: 1M x 768 fp32 cosine with labels; "
                    "4: KV-cache top-2048 (8 heads x 131k keys); 5: 1B x 128 uint8 with concurrent updates")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--n", type=int, default=0, help="rows (default: the config's)")
    ap.add_argument("--nq", type=int, default=10_000)
    ap.add_argument("--dim", type=int, default=0)
    ap.add_argument("--k", type=int, default=0)
    ap.add_argument("--batch", type=int, default=0)
    ap.add_argument("--cpu-queries", type=int, default=0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-defaults", action="store_true",
                    help="config 2: skip the second measurement with the API's defaults (id order, batch 2,048)")
    ap.add_argument("--lists", type=int, default=-1, help="k-means lists (default: the config's; 0: none)")
    ap.add_argument("--stride", type=int, default=0,
                    help="configs 2 and 3: the index's anchor stride (default: the API's, 16)")
    ap.add_argument("--probe", type=int, default=-1,
                    help="lists probed per query (default 0: the anchors of each query's 8 nearest lists set its threshold)")
    ap.add_argument("--summarize", nargs="+", metavar="DIR",
                    help="print a summary of the rocprofv3 CSV output under DIR (of a run with the "
                    "same --warmup and --steps) and exit; needs no GPU")
    ap.add_argument("--stamp", action="store_true",
                    help="print the sources stamp of the int8 screen (as traffic summaries record it) and exit")
    args = ap.parse_args()
    if args.summarize:
        print(summarize_profiles(args.summarize, args.warmup, args.steps))
        return
    if args.stamp:
        print(sources_stamp())
        return
    if args.gpus != 1:
        print(
            "bench.py measures one GPU: this build targets single-GPU boxes (the sharded search is a "
            "design, not code); run with --gpus 1",
            file=sys.stderr,
        )
        sys.exit(2)

    import libcertex_amd as certex
    from libcertex_amd import _capi as C

    C.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.config == 3:
        args.cpu_queries = args.cpu_queries or 16
        print(json.dumps(bench_config3(args)), flush=True)
        return
    if args.config == 4:
        args.cpu_queries = args.cpu_queries or 8
        print(json.dumps(bench_config4(args)), flush=True)
        return
    if args.config == 5:
        print(json.dumps(bench_config5(args)), flush=True)
        return
    args.cpu_queries = args.cpu_queries or 64
    args.batch = args.batch or 10_000
    n, d, nq, k = args.n or 10_000_000, args.dim or 128, args.nq, args.k or 10
    centres = torch.rand((1000, d), generator=torch.Generator().manual_seed(1), dtype=torch.float64) * 80.0
    centres = centres.float().to(dev)
    X = mixture_u8(n, d, 1000, centres, 2, dev)
    Q = mixture_u8(nq, d, 1000, centres, 3, dev)
    torch.cuda.synchronize()

    # the rows are stored in the order of 4,096 k-means lists that no search probes: the same
    # exhaustive screen, whose MFMA operands then change less from one row tile to the next
    n_lists = 4096 if args.lists < 0 else args.lists
    args.probe = 0 if args.probe < 0 else args.probe
    stride_kw = {"anchor_stride": args.stride} if args.stride > 0 else {}
    idx = certex.Index(d, metric="l2", n_lists=n_lists, **stride_kw)
    t_build = time.perf_counter()
    idx.add(X)
    torch.cuda.synchronize()
    t_build = time.perf_counter() - t_build

    def step():
        return idx.search(Q, k=k, batch=args.batch, probe_lists=args.probe)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    L = C.lib()
    C.check(L.cuvsCertexTimingBegin())
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        D, I = step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms = (ctypes.c_double * 4)()
    launches = (ctypes.c_int64 * 4)()
    C.check(L.cuvsCertexTimingEnd(ms, launches))
    ms_per_step = (t1 - t0) * 1000.0 / args.steps
    qps = nq / (ms_per_step / 1000.0)

    with certex.search_stats() as st:
        D, I = step()

    # roofline of the screen: 2 N d int8 ops per query
    screen_ms = ms[2] / max(1, launches[2])
    # the verify: every survivor's bucket entry (4 B) and its 128-byte code row, and the queries
    row_b = 128 if d <= 128 else 256
    verify_bytes = (st.survivors * (4 + row_b) + nq * row_b) / max(1, launches[3] // args.steps)
    phase_roofs = {"verify_topk": hbm_roofline(
        "verify_topk_i8_small_kernel (+ verify_topk_i8_kernel for buckets over 512)", verify_bytes,
        ms[3] / max(1, launches[3]),
        f"{st.survivors / max(1, st.queries):.1f} survivors x ({row_b} B code row + 4 B bucket "
        f"entry), plus the query, per query")}
    batches = (nq + args.batch - 1) // args.batch
    ops_per_launch = 2.0 * n * d * nq / batches
    achieved = ops_per_launch / (screen_ms / 1000.0) / 1e12
    clock = clock_fields(achieved, P_INT8_TOPS)
    phase_ms = {
        name: round(ms[i] / args.steps, 4) for i, name in enumerate(("anchors", "threshold", "screen", "verify_topk"))
    }

    # the same search with the API's defaults: an index in id order (no lists) and batches of
    # 2,048 queries; timed the same way, for the number a caller who changes nothing gets
    defaults = None
    if not args.no_defaults:
        plain = certex.Index(d, metric="l2")
        plain.add(X)

        def plain_step():
            return plain.search(Q, k=k)

        d_ms, d_phase, d_launch = timed_steps(plain_step, args.steps, args.warmup)
        d_screen = d_phase[2] / max(1, d_launch[2])
        d_ops = 2.0 * n * d * nq / max(1, d_launch[2] // args.steps)
        defaults = {"value": round(nq / (d_ms / 1000.0), 1), "ms_per_step": round(d_ms, 4),
                    "batch": 2048, "row_order": "id order (no lists)",
                    "screen_frac": round(d_ops / (d_screen / 1000.0) / 1e12 / P_INT8_TOPS, 4),
                    "phase_ms_per_step": {p: round(d_phase[i] / args.steps, 4) for i, p in enumerate(PHASES)}}
        del plain
        torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        import numpy as np

        import oracle

        Xh, Qh = X.cpu().numpy(), Q.cpu().numpy()
        cpu, cq, i_cpu = cpu_baseline(lambda c: oracle.knn(Xh, Qh[:c], k, "l2")[1], nq, args.cpu_queries,
                                      f"exhaustive fp64 against all {n} rows")
        cpu["sample"] += f"; ids equal to the GPU's: {bool(np.array_equal(i_cpu, I[:cq].cpu().numpy()))}"

    line = {
        "metric": "exact 10-NN queries/sec, 10M x 128 uint8 L2, 1 MI355X; screen % MFMA peak",
        "value": round(qps, 1),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (config 2 Gaussian mixture, torch generators seeded 1/2/3)",
        "config": {
            "workload": "config 2: exact 10-NN, L2, base 10,000,000 x 128 uint8, 10,000 queries",
            "n": n,
            "dim": d,
            "n_queries": nq,
            "k": k,
            "batch": args.batch,
            "anchor_stride": idx.anchor_stride,
            "n_lists": n_lists,
            "probe_lists": args.probe if n_lists else 0,
            "row_order": ("k-means list order" if n_lists else "id order")
            + (" (every row is screened; the lists order the stored rows, and the anchors of each query's"
               " 8 nearest lists bound its threshold)" if n_lists and not args.probe else ""),
            "build_s": round(t_build, 2),
            "screen": "int8 MFMA (exact), re-rank fp64",
            "phase_ms_per_step": phase_ms,
            "survivors_per_query": round(st.survivors / max(1, st.queries), 2),
            "phase_rooflines": phase_roofs,
            "api_defaults": defaults,
        },
        "roofline": {
            "bound": "mfma",
            "kernel": "screen_kernel<int8_rows,2,512,false,false,8,2,false> (int8 MFMA screen, 128-row steps)",
            "achieved": round(achieved, 2),
            "peak": P_INT8_TOPS,
            "unit": "TOP/s",
            "frac": round(achieved / P_INT8_TOPS, 4),
            # measured only for the default workload (profiles/screen_i8_c2_traffic.txt)
            "traffic": screen_traffic()
            if (n, d, nq, args.batch, n_lists, args.probe, idx.anchor_stride)
            == (10_000_000, 128, 10_000, 10_000, 4096, 0, 16) else None,
            "avg_launch_ms": round(screen_ms, 4),
            "ops_per_launch": ops_per_launch,
            **clock,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
