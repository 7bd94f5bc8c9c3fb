"""Benchmark of the MI355X Groth16 prover core (BASELINE.json metric:
"Groth16 prove ms at 2^16 constraints; G1 MSM Mpoints/s at 2^20").

A step is one G1 MSM over 2^20 points (P_i = k_i G1 for
seeded k_i, scalars uniform in [0, r)), with points and scalars resident in
HBM.  `value` is that MSM's throughput in Mpoints/s.  The same run also times
full Groth16 proves, each checked by the product's verifier:
  prove_2_16            config 4's statement (62.7 k constraints, domain 2^16),
                        built by the reference's own statement builder and
                        committed under tests/golden/statements
  prove_config1         config 1's quantized MLP statement (domain 2^13)
  prove_2_16_synthetic  a uniform-witness config-5-shaped R1CS, domain 2^16
  prove_2_22_config5    config 5 at its full 2^22 constraints
the 2^22 NTT of config 2, and the CPU oracle's restatement of the reference
MSM on the host cores (cpu_baseline).  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "cuda-zkml_amd"))
sys.path.insert(0, os.path.join(ROOT, "tests"))

# MI355X peaks: full-rate 32-bit mad (v_mad_u64_u32 issues at the VALU rate on
# gfx950, measured) = 256 CU x 64 lanes x 2.4 GHz; HBM3E 8 TB/s.
PEAK_MAD_TOPS = 256 * 64 * 2.4e9 / 1e12
PEAK_HBM_GBS = 8000.0
R_ORDER = 0x30644E72E131A029B85045B68181585D2833E84879B9709143E1F593F0000001
MADS_PER_FIELD_MUL = 136  # 8x32-bit CIOS: 2*8^2 + 8


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def msm_algorithmic_mults(n, c):
    """BASELINE.md F(N) with W = ceil(255/c) signed windows."""
    w = -(-255 // c)
    return n * w * 10 + w * (1 << (c - 1)) * 2 * 14 + w * (6 * c + 14)


def best_c(n):
    return min(range(8, 22), key=lambda c: msm_algorithmic_mults(n, c))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--log-n", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prove", action="store_true")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (torch's copy kernel), the reference for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    args = ap.parse_args()
    if args.copy_calibration:
        import torch
        nbytes = args.copy_calibration << 20
        a = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
        b = torch.empty_like(a)
        for _ in range(3):
            b.copy_(a)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": nbytes, "copy_bytes_written": nbytes, "launches": 3}), flush=True)
        return
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        sys.exit(2)

    import zkml_amd
    ctx = zkml_amd.Context(0)
    rng = np.random.default_rng(20260601)
    n = 1 << args.log_n

    # ---------------- MSM 2^20 (the step)
    log(f"[bench] generating {n} points P_i = k_i G1 on the GPU")
    k = zkml_amd.random_fr(n, rng)
    s = zkml_amd.random_fr(n, rng)
    dk = ctx.upload(k)
    dp = ctx.alloc(n * 64)
    ctx.g1_generator_mul(dk, n, dp)
    ds = ctx.upload(s)
    ctx.sync()
    for _ in range(args.warmup):
        res = ctx.msm_g1(dp, ds, n)
    ctx.sync()
    ctx.set_profiling(True)
    ctx.reset_kernel_stats()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = ctx.msm_g1(dp, ds, n)
    ctx.sync()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    kernels = {}
    for name in ctx.kernel_names():
        cnt, ms = ctx.kernel_stats(name)
        kernels[name] = {"ms_per_step": ms / args.steps, "launches_per_step": cnt / args.steps}
    ctx.set_profiling(False)
    mpoints = n / (ms_step * 1e-3) / 1e6
    log(f"[bench] MSM 2^{args.log_n}: {ms_step:.3f} ms/step, {mpoints:.1f} Mpoints/s")

    # roofline of the dominant kernel (bucket accumulation): every sorted
    # (window, point) entry costs one mixed XYZZ addition = 10 field mults.
    c, windows = zkml_amd.Context.msm_config(n)
    acc = kernels.get("msm_accumulate", {"ms_per_step": float("nan"), "launches_per_step": 1})
    acc_ms = acc["ms_per_step"] / max(acc["launches_per_step"], 1)
    acc_mads = n * windows * 10 * MADS_PER_FIELD_MUL
    achieved = acc_mads / (acc_ms * 1e-3) / 1e12
    # HBM bytes per launch of the same kernel, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE runs (profiles/msm_2e20_pmc_traffic.md), scaled by
    # the counters' reading for a plain copy of known size
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "msm_2e20_pmc_traffic.json")
    if args.log_n == 20 and os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("msm_accumulate_bytes_per_launch")
    # whole-MSM VALU fraction with BASELINE.md's algorithmic count
    f_mults = msm_algorithmic_mults(n, best_c(n))
    msm_frac = f_mults * MADS_PER_FIELD_MUL / (ms_step * 1e-3) / 1e12 / PEAK_MAD_TOPS

    # ---------------- NTT 2^22 (config 2)
    ntt = {}
    ln = 22
    a = zkml_amd.random_fr(1 << ln, rng)
    da = ctx.upload(a)
    do = ctx.alloc((1 << ln) * 32)
    ctx.ntt(do, da, ln)
    ctx.sync()
    ctx.set_profiling(True)
    ctx.reset_kernel_stats()
    reps = 10
    t0 = time.perf_counter()
    for _ in range(reps):
        ctx.ntt(do, da, ln)
    ctx.sync()
    wall = (time.perf_counter() - t0) * 1e3 / reps
    _, kms = ctx.kernel_stats("ntt_pass")
    ctx.set_profiling(False)
    kms /= reps
    ntt = {"log_n": ln, "ms": round(kms, 4), "wall_ms": round(wall, 4),
           "hbm_GBps_alg": round(64 * (1 << ln) / (kms * 1e-3) / 1e9, 1),
           "hbm_frac": round(64 * (1 << ln) / (kms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
           "valu_frac": round(((1 << ln) // 2 * ln) * MADS_PER_FIELD_MUL / (kms * 1e-3) / 1e12 / PEAK_MAD_TOPS, 4)}
    log(f"[bench] NTT 2^22: {kms:.3f} ms")
    del da, do

    # ---------------- full prove at 2^16
    prove = prove_syn = prove22 = prove_c1 = None
    if not args.no_prove:
        import tempfile
        from statements import load as load_statement

        def prove_case(stmt, reps, label):
            """GPU setup, then `reps` proves of a statement (nc, nv, npub, A, B, C,
            w) with the witness handed over from host memory; the proof is
            checked with the product's verifier."""
            nc, nv, npub, A, B, C, w = stmt
            log(f"[bench] {label}: {nc} constraints, GPU setup")
            r = ctx.r1cs(nc, nv, npub, A, B, C)
            with tempfile.TemporaryDirectory() as td:
                t0 = time.perf_counter()
                ctx.setup(r, 0xDEADBEEF42, os.path.join(td, "pk.bin"), os.path.join(td, "vk.bin"))
                t_setup = time.perf_counter() - t0
                pk = ctx.load_pk(os.path.join(td, "pk.bin"))
                vk_bytes = open(os.path.join(td, "vk.bin"), "rb").read()
            ctx.prove(pk, r, w, npub, 0xCAFEBABE)  # warm-up (workspaces, plans)
            times, parts, proof = [], None, None
            for _ in range(reps):
                t0 = time.perf_counter()
                proof, t = ctx.prove(pk, r, w, npub, 0xCAFEBABE)
                times.append((time.perf_counter() - t0) * 1e3)
                parts = t
            pub = np.zeros((npub, 4), dtype=np.uint64)
            for i in range(npub):  # w[1..npub] to standard form for the verifier
                x = sum(int(w[1 + i][k]) << (64 * k) for k in range(4)) * pow(1 << 256, -1, R_ORDER) % R_ORDER
                pub[i] = [(x >> (64 * k)) & (2**64 - 1) for k in range(4)]
            ok = zkml_amd.verify(vk_bytes, proof, pub)
            out = {"constraints": nc, "variables": nv, "public": npub, "domain": 1 << r.log_n,
                   "ms": round(float(np.median(times)), 3), "setup_s": round(t_setup, 2), "proof_verifies": ok,
                   "breakdown_ms": {k_: round(v, 3) for k_, v in parts.items()}}
            log(f"[bench] {label}: {out['ms']:.3f} ms (median of {reps}), setup {t_setup:.1f} s, verifies: {ok}")
            pk.close()
            r.close()
            return out

        def synthetic(nc, seed):
            A, B, C, w = zkml_amd.synthetic_r1cs(nc, 4, 16, seed)
            return nc, w.shape[0], 4, A, B, C, w

        def fixture(name):
            nc, nv, npub, _npriv, A, B, C, w = load_statement(name)
            return nc, nv, npub, A, B, C, w

        prove = prove_case(fixture("config4"), 7, "prove config 4 (2^16)")
        prove_c1 = prove_case(fixture("config1"), 7, "prove config 1 (2^13)")
        prove_syn = prove_case(synthetic((1 << 16) - 64, 16), 5, "prove 2^16 synthetic")
        prove22 = prove_case(synthetic(1 << 22, 22), 3, "prove 2^22 (config 5)")

    # ---------------- CPU baseline (oracle restatement of the reference MSM)
    cpu = None
    if not args.no_cpu:
        from bindings import oracle, ptr
        lib = oracle()
        sample = 1 << 18
        pts = ctx.d2h(dp, (n, 8))[:sample].copy()
        sc = np.ascontiguousarray(s[:sample])
        out = np.zeros(8, dtype=np.uint64)
        threads = 1
        t0 = time.perf_counter()
        lib.orc_msm_g1(ptr(pts), ptr(sc), sample, 0, threads, ptr(out))
        dt = time.perf_counter() - t0
        cpu = {"value": round(sample / dt / 1e6, 4), "unit": "Mpoints/s", "cores": threads, "kind": "port",
               "sample": f"G1 MSM over the first 2^18 of the same points/scalars, reference Pippenger "
                         f"(MSMConfig windows, Jacobian mixed adds, serial running sums), {dt:.2f} s"}
        log(f"[bench] CPU baseline: {cpu['value']} Mpoints/s ({dt:.2f} s)")

    line = {
        "metric": "Groth16 prove ms at 2^16 constraints; G1 MSM Mpoints/s at 2^20",
        "value": round(mpoints, 2),
        "unit": "Mpoints/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32 (BN254 Fq/Fr 256-bit modular, 9x29-bit limbs)",
        "data": "synthetic, seeded (P_i = k_i G1, k_i and s_i uniform in [0, r))",
        "config": {"workload": f"G1 MSM, n = 2^{args.log_n}, BASELINE config 3 (uniform scalars)",
                   "window_bits": c, "windows": windows},
        "roofline": {"bound": "valu", "achieved": round(achieved, 3), "peak": round(PEAK_MAD_TOPS, 2),
                     "unit": "T mad32/s", "frac": round(achieved / PEAK_MAD_TOPS, 4), "traffic": traffic,
                     "kernel": "msm_accumulate", "kernel_ms": round(acc_ms, 4)},
        "msm_valu_frac_whole": round(msm_frac, 4),
        "kernels_ms_per_step": {k_: round(v["ms_per_step"], 4) for k_, v in kernels.items()},
        "prove_2_16": prove,
        "prove_2_16_synthetic": prove_syn,
        "prove_config1": prove_c1,
        "prove_2_22_config5": prove22,
        "ntt_2_22": ntt,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
