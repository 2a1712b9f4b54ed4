"""Benchmark: KMeans Lloyd iterations/s on one MI355X.

Workload: 500,000 x 100 fp32 from 50 isotropic Gaussian blobs (centres
~U[-10,10]^100, sigma 1), k = 50, seeded random-row init -- the shape of
skmetal's README headline.  A "step" is one Lloyd iteration (fused E-step and
per-cluster sums, finalize) over all 500,000 rows, with X already resident in
HBM.  The arithmetic is fp32-equivalent: x and c enter as an exact three-part
bf16 split (x = hi + mid + lo, every fp32 value represented exactly), the
products of the parts are exact in the fp32 accumulators of the bf16 MFMAs,
the sums use all three parts and the E-step 6 of the 9 part products (the
three left out total at most 2^-23 |x_i c_i| per feature).  The same steps on
the fp32-MFMA kernel are timed beside it.  The measurements reported beside
the metric (that fp32-MFMA run, the end-to-end estimator fit, the k-means++
seeding and skmetal's k-means|| seeding) run first; then the headline handle runs the W warm-up steps and the
K timed steps from the seeded initial centres.  The steps are timed with HIP
events on the library's stream (skmetal_hip_lloyd_iterate).  The same steps
are then run again from the same initial centres with each step's kernels
bracketed by HIP events on that stream: the dominant kernel's average launch
time over those steps gives its roofline fraction.

cpu_baseline: scikit-learn's KMeans(algorithm="lloyd") -- the CPU
implementation skmetal routes KMeans to -- on the same workload, same init, on
this machine's cores; per-iteration time from fits of N and 1 iterations.

Prints one JSON line.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_BF16_MFMA_TFLOPS = 2500.0
PEAK_HBM_GBPS = 8000.0


def _traffic_from_profile(name: str):
    """HBM bytes per assign launch, from the committed rocprofv3 PMC summary."""
    p = ROOT / "profiles" / name
    if not p.exists():
        return None
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", p.read_text())
    return float(m.group(1)) if m else None


MFMA_16x16x32_FLOP = 2 * 16 * 16 * 32


def fused3_mfma_per_tile(k: int, d: int):
    """v_mfma_f32_16x16x32_bf16 instructions of k_fused3 (split_kernels.hip,
    Fused3Geom and the E-step / sums waves): (per 16-row half tile in the
    E-step, per 32-row tile in the sums).  ld = d rounded up to 4; NK 32-feature
    K steps and a tail of 4 or 16 features.  E-step: per 16-centre block six
    part products per K step (hh, mh, lh, hm, mm, hl) and 1 (tail 4) or 3
    (tail 16) tail MFMAs; a last block of at most 4 centres is stacked (three
    MFMAs per K step for all nine products, 1 or 2 tail MFMAs).  Sums: per
    centre block and 16-feature block, one MFMA per part (the tail-4 block
    packs its three parts into one)."""
    ld = -(-d // 4) * 4
    nk, tail = ld // 32, ld % 32
    cb = -(-k // 16)
    nt = {0: 0, 4: 1, 16: 3}[tail]
    nts = {0: 0, 4: 1, 16: 2}[tail]
    stacked = k - 16 * (cb - 1) <= 4
    e16 = (cb - 1) * (6 * nk + nt) + ((3 * nk + nts) if stacked else (6 * nk + nt))
    nfb = (32 * nk + (16 if tail else 0)) // 16
    s32 = cb * (3 * (nfb - 1) + 1) if tail == 4 else cb * 3 * nfb
    return e16, s32


def copy_probe(mib: int) -> None:
    """One device-to-device copy of `mib` MiB (hipMemcpy), a known-size kernel the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters are calibrated against."""
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so.7")  # the runtime libskmetal_hip.so already loaded
    nbytes = ctypes.c_size_t(mib << 20)
    a, b = ctypes.c_void_p(), ctypes.c_void_p()
    assert hip.hipMalloc(ctypes.byref(a), nbytes) == 0 and hip.hipMalloc(ctypes.byref(b), nbytes) == 0
    assert hip.hipMemset(a, 1, nbytes) == 0
    assert hip.hipMemcpy(b, a, nbytes, 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipDeviceSynchronize() == 0
    hip.hipFree(a)
    hip.hipFree(b)


def cpu_baseline(X, C0, iters: int, reps: int = 3):
    """sklearn Lloyd on this host: seconds per iteration (median of reps)."""
    try:
        import sklearn
        from sklearn.cluster import KMeans
    except ImportError:  # pragma: no cover - sklearn is part of the image
        return None
    cores = len(os.sched_getaffinity(0))

    def fit(m):
        km = KMeans(n_clusters=C0.shape[0], init=C0, n_init=1, max_iter=m, tol=0.0, algorithm="lloyd")
        t = time.perf_counter()
        km.fit(X)
        return time.perf_counter() - t, km.n_iter_

    per = []
    for _ in range(reps):
        tn, it_n = fit(iters)
        t1, _ = fit(1)
        per.append((tn - t1) / (it_n - 1) if it_n == iters and iters > 1 else tn / it_n)
    s = float(np.median(per))
    return dict(
        value=1.0 / s,
        unit="Lloyd iters/s",
        cores=cores,
        kind="reference",
        sample=(f"sklearn {sklearn.__version__} KMeans(algorithm='lloyd', init=same {C0.shape[0]} rows, n_init=1, "
                f"tol=0) on the full {X.shape[0]}x{X.shape[1]} workload; per-iteration time = "
                f"(t_fit(max_iter={iters}) - t_fit(max_iter=1))/({iters}-1), median of {reps}; "
                f"OMP threads={os.environ.get('OMP_NUM_THREADS', 'default')}"),
    )


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--workload", default="c2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the sklearn CPU baseline")
    ap.add_argument("--cpu-iters", type=int, default=8)
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MIB",
                    help="also run one device-to-device copy of MIB MiB (counter calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: one GPU per run; --gpus {args.gpus} is not supported "
              "(the library shards nothing across GPUs).", file=sys.stderr)
        sys.exit(2)

    from skmetal_amd import _bridge, _synth

    if not _bridge.HIP_AVAILABLE:
        raise SystemExit(f"GPU path unavailable: {_bridge.last_error()}")
    wl = _synth.WORKLOADS[args.workload]
    X, C0 = _synth.generate(args.workload, seed=0)
    n, d = X.shape
    k = C0.shape[0]

    # The measurements reported beside the metric run first, on their own
    # handles and on the headline handle's resident X; the headline's W
    # warm-up steps and K timed steps follow them on that handle.
    h = _bridge.LloydHandle(n, d, k)
    try:
        t = time.perf_counter()
        h.load(X, center=True)
        h2d_s = time.perf_counter() - t
        # the same fixed-iteration run on the fp32-MFMA kernel (v_mfma_f32_4x4x1,
        # per-cluster sums by a VALU walker)
        os.environ["SKMETAL_HIP_SPLIT"] = "0"
        try:
            with _bridge.LloydHandle(n, d, k) as h32:
                h32.load(X, center=True)
                h32.set_centers(C0)
                h32.iterate(args.warmup)
                h32.set_centers(C0)
                ms32 = h32.iterate(args.steps)
                fp32_mode = h32.info()
        finally:
            del os.environ["SKMETAL_HIP_SPLIT"]
        fit_ms = pp_ms = kpar_ms = None
        if args.workload == "c2":
            # the whole estimator fit a user runs on this X (validation,
            # tolerance, upload, k-means++, Lloyd to convergence, final
            # E-step): median of 3 after a warm-up
            from sklearn.cluster import KMeans

            import skmetal_amd

            def _fit_once():
                t0 = time.perf_counter()
                skmetal_amd.accelerate(KMeans(n_clusters=k, init="k-means++", n_init=1, random_state=0)).fit(X)
                return time.perf_counter() - t0

            _fit_once()
            fit_ms = round(sorted(_fit_once() for _ in range(3))[1] * 1e3, 2)
            # k-means++ seeding of the resident X on the device with
            # scikit-learn's draws for random_state=0 (KMeans(init="k-means++")
            # runs it once per fit)
            T, first, u = _bridge.plusplus_draws(np.random.RandomState(0), n, k)
            h.plusplus_with(T, first, u)
            t = time.perf_counter()
            h.plusplus_with(T, first, u)
            pp_ms = round((time.perf_counter() - t) * 1e3, 3)
            # skmetal's own MetalKMeans seeding (k-means||: max(1, int(2 + ln k))
            # rounds of distances, numpy's weighted draws and the prune, all on
            # the device) of the resident X for random_state=0
            import warnings

            from sklearn.exceptions import ConvergenceWarning

            from skmetal_amd.estimators.cluster import kmeans_parallel_init

            with warnings.catch_warnings():
                warnings.simplefilter("ignore", ConvergenceWarning)
                kmeans_parallel_init(X, k, np.random.RandomState(0), h)
                t = time.perf_counter()
                kmeans_parallel_init(X, k, np.random.RandomState(0), h)
                kpar_ms = round((time.perf_counter() - t) * 1e3, 3)
        # the headline: W warm-up steps, then K timed steps from the same
        # initial centres
        h.set_centers(C0)
        h.iterate(args.warmup)
        h.set_centers(C0)
        t = time.perf_counter()
        ms = h.iterate(args.steps)
        wall = time.perf_counter() - t
        # the same steps again from the same centres, each kernel bracketed by
        # HIP events (a marker costs a few microseconds of queue time, so the
        # step time above is measured without them)
        h.set_centers(C0)
        _, (ms_assign, ms_update, ms_final) = h.iterate(args.steps, kernel_times=True)
        mode = h.info()
    finally:
        h.close()
    if args.calib_copy:
        copy_probe(args.calib_copy)

    step_s = ms / 1e3 / args.steps
    it_s = 1.0 / step_s
    flops = 2.0 * n * k * d
    assign_s = ms_assign / 1e3
    fused, split, asplit = mode["fused"], mode["split"], mode["asplit"]
    kname = "k_fused3" if split else "k_fused" if fused else "k_assign3" if asplit else "k_assign"
    traffic = _traffic_from_profile(f"{kname}_{args.workload}_pmc.txt")
    if split:
        # The binding roof of the assign work: its arithmetic intensity
        # 2nkd / (4nd + 4n + 4kd) -- X read once, the labels written, the
        # centres read -- against the fp32 ridge 157.3 TFLOP/s / 8 TB/s
        # = 19.7 flop/B.  At or above the ridge the fp32 MFMA roof binds
        # (2nkd / 157.3 TFLOP/s), below it HBM.  The other roof and the
        # kernel's bf16 MFMA instructions (fused3_mfma_per_tile) against the
        # bf16 peak are reported beside it.
        nbytes = 4.0 * n * d + 4.0 * n + 4.0 * k * d
        ai = flops / nbytes
        ridge = PEAK_FP32_MFMA_TFLOPS * 1e12 / (PEAK_HBM_GBPS * 1e9)
        e16, s32 = fused3_mfma_per_tile(k, d)
        bf16_flops = -(-n // 32) * (2 * e16 + s32) * MFMA_16x16x32_FLOP
        hbm_gbps = nbytes / assign_s / 1e9
        fp32_tflops = flops / assign_s / 1e12
        on_mfma = ai >= ridge
        roofline = {
            "kernel": ("k_fused3: E-step (||c||^2 - 2 x.c) + argmin + per-cluster sums, bf16 MFMAs over the exact "
                       "three-part split, fp32 accumulation"),
            "bound": "mfma" if on_mfma else "hbm",
            "achieved": round(fp32_tflops, 2) if on_mfma else round(hbm_gbps, 1),
            "peak": PEAK_FP32_MFMA_TFLOPS if on_mfma else PEAK_HBM_GBPS,
            "unit": "TFLOP/s" if on_mfma else "GB/s",
            "frac": round(fp32_tflops / PEAK_FP32_MFMA_TFLOPS if on_mfma else hbm_gbps / PEAK_HBM_GBPS, 4),
            "traffic": traffic,
            "roof": ("fp32 MFMA: 2nkd fp32-equivalent distance flops per launch" if on_mfma
                     else "HBM: 4nd + 4n + 4kd bytes per launch"),
            "arithmetic_intensity": round(ai, 2),
            "ridge": round(ridge, 2),
            "kernel_us": round(assign_s * 1e6, 2),
            "algorithmic_bytes": nbytes,
            "hbm_gbps": round(hbm_gbps, 1),
            "hbm_frac": round(hbm_gbps / PEAK_HBM_GBPS, 4),
            "fp32_equiv_tflops": round(fp32_tflops, 2),
            "fp32_mfma_frac": round(fp32_tflops / PEAK_FP32_MFMA_TFLOPS, 4),
            "bf16_mfma_tflops": round(bf16_flops / assign_s / 1e12, 1),
            "bf16_mfma_frac": round(bf16_flops / assign_s / 1e12 / PEAK_BF16_MFMA_TFLOPS, 4),
            "mfma_per_32_rows": {"e_step": 2 * e16, "sums": s32},
        }
    elif asplit:
        # MFMA roofline of the split E-step: six bf16 products per x.c term,
        # over the padded centres (multiples of 16 per pass) and features (32)
        kp = -(-k // (16 * (4 if k <= 64 else 8 if k <= 128 else 16))) * (16 * (4 if k <= 64 else 8 if k <= 128 else 16))
        dp = -(-d // 32) * 32
        mflops = 6.0 * 2.0 * n * kp * dp
        roofline = {
            "kernel": "k_assign3: ||c||^2 - 2 x.c on bf16 MFMAs over the exact three-part split + argmin",
            "bound": "mfma",
            "achieved": round(mflops / assign_s / 1e12, 1),
            "peak": PEAK_BF16_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(mflops / assign_s / 1e12 / PEAK_BF16_MFMA_TFLOPS, 4),
            "traffic": traffic,
            "fp32_equiv_tflops": round(flops / assign_s / 1e12, 2),
        }
    else:
        achieved = flops / assign_s / 1e12
        roofline = {
            "kernel": (f"{kname}: ||c||^2 - 2 x.c on fp32 MFMA + argmin"
                       + (" + per-cluster sums" if fused else "")),
            "bound": "mfma",
            "achieved": round(achieved, 2),
            "peak": PEAK_FP32_MFMA_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_FP32_MFMA_TFLOPS, 4),
            "traffic": traffic,
        }

    cpu = None if args.no_cpu else cpu_baseline(X, C0, args.cpu_iters)

    out = {
        "metric": "Lloyd iters/s + dist-evals/s at 500k x100,k=50 fp32; % of roofline",
        "value": round(it_s, 2),
        "unit": "Lloyd iters/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_s * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": f"KMeans Lloyd {n}x{d} fp32, k={k}, {wl.description}, seeded random-row init, "
                               f"fixed iterations (no convergence stop)",
                   "n": n, "d": d, "k": k},
        "dist_evals_per_s": round(n * k * it_s, 1),
        "wall_s_timed": round(wall, 4),
        "h2d_s": round(h2d_s, 4),
        "step_mode": (f"fused: {kname} (E-step + per-cluster sums) + k_finalize_reloc (finalize and in-stream "
                      "empty-cluster relocation in one launch; the relocation returns at once when no cluster "
                      "is empty)" if fused
                      else f"{kname} + sorted update + k_finalize_recs + k_reloc + k_finalize_loop"),
        "e_step": ("fp32-equivalent: exact three-part bf16 split of x and c (x = hi + mid + lo), 6 of 9 part "
                   "products on v_mfma_f32_16x16x32_bf16, fp32 accumulation; the 3 left out total <= 2^-23 |x_i c_i|"
                   if (split or (asplit and not fused)) else "fp32 MFMA (v_mfma_f32_4x4x1_16b_f32)"),
        "m_step": ("fp32: one-hot x each of the three exact bf16 parts on v_mfma_f32_16x16x32_bf16, fp32 "
                   "accumulation per block, fp64 across blocks" if split
                   else "fp32 VALU sums per block, fp64 across blocks"),
        "fp32_mfma_path": {"value": round(args.steps / (ms32 / 1e3), 2), "unit": "Lloyd iters/s",
                           "ms_per_step": round(ms32 / args.steps, 5),
                           "kernel": "k_fused" if fp32_mode["fused"] else "k_assign"},
        "partials": mode["partials"],
        "kernels_ms": ({kname: round(ms_assign, 5), "k_finalize_reloc": round(ms_final, 5)} if fused
                       else {kname: round(ms_assign, 5), "update": round(ms_update, 5),
                             "finalize": round(ms_final, 5)}),
        "roofline": roofline,
        "kmeans_plusplus_ms": pp_ms,
        "kmeans_parallel_init_ms": kpar_ms,
        "fit_kmeanspp_ms": fit_ms,
        "cpu_baseline": cpu,
    }
    if cpu:
        out["speedup_vs_cpu"] = round(it_s / cpu["value"], 1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
