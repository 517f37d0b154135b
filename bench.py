"""Key-switch throughput on one MI355X: the hoisted rotation batch of a CoeffToSlot BSGS stage.

Workload (the largest single-GPU configuration the metric is quoted on): one ciphertext at N = 2^16, L = 30 limbs of
31-bit primes, dnum 3 (10 limbs per digit), 6 special primes; ModUp once, then key switches to the rotation steps
{1..16, 32, 64, ..., 2^15}. 2^15 = N/2 is the identity (g = 1, a copy), so R = 26 switches. Keys: a regenerated in the
dot kernel from each key's ChaCha12 seed, b stored as dense 32-bit words (--bits 31: bit-packed, the reference's
PackedSeeded layout, which saves 3% of b at 31-bit primes); keys generated on the device from a synthetic ternary secret (h = 192) and Gaussian errors (sigma 3.19), the
ciphertext uniform. One "step" = the whole batch (ModUp + 26 dots + 26 ModDowns), inputs resident in HBM.

Prints one JSON line: value = key switches per second; roofline = the dominant stage's algorithmic bytes per launch
over its live average launch time (HIP events on its stream); ks_roofline = the batch's algorithmic bytes over the
step time; cpu_baseline = the oracle (this repository's C++ restatement of the reference's CPU twin) on a bounded
sample of the same batch on this host's cores.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBPS = 8000.0
STEPS_SET = list(range(1, 17)) + [1 << k for k in range(5, 16)]


def key_bytes_rows(ch, bits):
    """Rows of algorithmic traffic (words of N): E = D (l + k); b counted at its stored width."""
    L, k, D = len(ch.q), len(ch.p), ch.dnum
    E = D * (L + k)
    beta = (bits or 32) / 32.0
    return dict(
        E=E,
        modup=3 * E,  # INTT 2l, conversion l + (E - l), NTT 2 (E - l)
        dot=E + E * beta + L + 2 * (L + k),
        md_intt=4 * k,
        md_bconv=2 * k + 2 * L,
        md_ntt=6 * L,
        ks=E * (1 + beta) + 11 * L + 8 * k,  # one hoisted key switch (dot + ModDown)
        single=4 * E + E * beta + 11 * L + 8 * k,  # a key switch with its own ModUp
        floor=4 * L + E * beta,
    )


def cpu_baseline(ch, ct, top, keys_host, gals, budget_s=20.0):
    """The oracle's hoisted batch on this host: threads = min(cores, 16) (one thread per core, as the reference's
    host pool, crates/pc-hostrt/src/lib.rs:176-226); the sample grows until about budget_s of work."""
    from tests import twin

    cores = min(os.cpu_count() or 1, 16)
    twin.set_threads(cores)
    oc = twin.Ctx(ch.logn, ch.q, ch.p, ch.dnum)
    seeds = np.stack([k[0] for k in keys_host])
    bs = [k[1] for k in keys_host]
    live = [i for i, g in enumerate(gals) if g != 1]
    r = 2
    t = 0.0
    while True:
        sel = live[:r]
        t0 = time.perf_counter()
        outs = oc.rotate_hoisted(ct, top, seeds[sel], [bs[i] for i in sel], [gals[i] for i in sel])
        t = time.perf_counter() - t0
        if r >= len(live) or t * (len(live) / r) > budget_s:
            break
        r = len(live)
    return dict(value=r / t, unit="key-switches/s", cores=cores, kind="port",
                sample=f"ModUp + {r} hoisted key switches of the same batch (a regenerated per call, cold), {t:.2f} s"), outs, sel


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--bits", type=int, default=0, help="stored width of key b (0 = dense 32-bit words)")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for {args.gpus})", file=sys.stderr)
        sys.exit(2)

    import perseus_amd as pa

    if pa.device_count() < 1:
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    ch = pa.preset("c3")
    n, top = ch.n, len(ch.q) - 1
    gals = [pow(5, s % (n // 2), 2 * n) for s in STEPS_SET]
    R = sum(1 for g in gals if g != 1)
    rng = np.random.default_rng(2024)
    ctx = pa.Context(ch, k_rot=R)
    # synthetic key material: ternary secret of weight 192, Gaussian errors, ChaCha seeds
    secret = np.zeros(n, np.int8)
    pos = rng.choice(n, 192, replace=False)
    secret[pos] = rng.choice([-1, 1], 192)
    seeds = rng.integers(0, 1 << 32, (len(gals), 8), dtype=np.uint64).astype(np.uint32)
    errors = np.clip(np.round(rng.normal(0, 3.19, (len(gals), ch.dnum, n))), -45, 45).astype(np.int64)
    keys = pa.Keys(ctx, gals, seeds=seeds, bits=args.bits, secret=secret, errors=errors)
    ct = np.zeros((2, ch.rows, n), np.uint32)
    for part in range(2):
        for t in range(top + 1):
            ct[part, t] = rng.integers(0, ch.primes[t], n)
    st = pa.Stream()
    dev = pa.DevBuf.from_array(ct)
    outs = ctx.ct_buf(len(gals))
    idx = list(range(len(gals)))

    for _ in range(args.warmup):
        ctx.rotate_hoisted(keys, idx, dev, top, outs, st)
    st.sync()
    pa.check(pa.LIB.pc_hip_device_sync(), "sync")
    ctx.timing(16 * args.steps)
    e0, e1 = pa.Event(), pa.Event()
    t0 = time.perf_counter()
    e0.record(st)
    for _ in range(args.steps):
        ctx.rotate_hoisted(keys, idx, dev, top, outs, st)
    e1.record(st)
    st.sync()
    pa.check(pa.LIB.pc_hip_device_sync(), "sync")
    wall = time.perf_counter() - t0
    ctx.timing(0)
    dev_ms = e0.elapsed_ms(e1) / args.steps
    ms = wall * 1e3 / args.steps
    stages = ctx.timing_read()

    rows = key_bytes_rows(ch, args.bits)
    row_bytes = 4 * n
    per_launch_rows = {"dot": R * rows["dot"], "md_intt": R * rows["md_intt"], "md_bconv": R * rows["md_bconv"],
                       "md_ntt": R * rows["md_ntt"], "modup_intt": 2 * len(ch.q),
                       "modup_bconv": len(ch.q) + (rows["E"] - len(ch.q)), "modup_ntt": 2 * (rows["E"] - len(ch.q))}
    stage_info = {}
    for name, (tot, cnt) in stages.items():
        if cnt:
            avg = tot / cnt
            gbps = per_launch_rows[name] * row_bytes / (avg * 1e-3) / 1e9
            stage_info[name] = {"avg_ms": round(avg, 4), "launches": cnt, "GBps": round(gbps, 1)}
    dom = max(stage_info, key=lambda k: stage_info[k]["avg_ms"] * stage_info[k]["launches"])
    kernel_names = {"dot": "dot_k (ks_dot_key)", "md_ntt": "fwd_cols + fwd_rows (ModDown NTT + epilogue)",
                    "md_intt": "inv_rows + inv_cols (ModDown INTT)", "md_bconv": "bconv_k (ModDown)",
                    "modup_intt": "inv_rows + inv_cols (ModUp INTT)", "modup_bconv": "bconv_k (ModUp)",
                    "modup_ntt": "fwd_cols + fwd_rows (ModUp NTT)"}
    achieved = stage_info[dom]["GBps"]
    traffic = None
    roofline = {"bound": "hbm", "kernel": kernel_names[dom], "achieved": achieved, "peak": HBM_PEAK_GBPS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBPS, 4),
                "algorithmic_bytes_per_launch": per_launch_rows[dom] * row_bytes, "traffic": traffic}
    hoist_bytes = (rows["modup"] + R * rows["ks"]) * row_bytes
    ks_gbps = hoist_bytes / (ms * 1e-3) / 1e9
    value = R / (ms * 1e-3)
    out = {
        "metric": "key-switches/sec at N=2^16 (% HBM roofline)",
        "value": round(value, 1),
        "unit": "key-switches/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "device_ms_per_step": round(dev_ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32",
        "data": "synthetic",
        "config": {"workload": "hoisted rotation batch (CoeffToSlot BSGS)", "N": n, "L": len(ch.q), "dnum": ch.dnum,
                   "special_primes": len(ch.p), "prime_bits": 31, "rotation_steps": STEPS_SET,
                   "key_switches_per_step": R, "key_b_bits": args.bits, "key_a": "regenerated in-kernel (ChaCha12)"},
        "roofline": roofline,
        "ks_roofline": {"bound": "hbm", "achieved": round(ks_gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                        "frac": round(ks_gbps / HBM_PEAK_GBPS, 4), "algorithmic_bytes_per_step": hoist_bytes,
                        "ks_per_s_at_peak": round(R / (hoist_bytes / (HBM_PEAK_GBPS * 1e9)), 1)},
        "stages": stage_info,
    }
    if not args.no_cpu:
        host_keys = [(seeds[i], keys.download_b(i)) for i in idx]
        cpu, cpu_outs, sel = cpu_baseline(ch, ct, top, host_keys, gals)
        out["cpu_baseline"] = cpu
        # the GPU outputs of the sampled keys, word for word against the oracle's
        got = outs.download((len(gals), 2, ch.rows, n))
        out["cpu_gpu_bit_exact"] = bool(all((got[i, :, : top + 1] == cpu_outs[j][:, : top + 1]).all()
                                            for j, i in enumerate(sel)))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
