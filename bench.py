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
  prove_config4_named   config 4's network as written (1x8x8 input, four 3x3
                        filters, MLP 144 -> 32 -> 10, private model and input
                        under Poseidon, routing): 707 k constraints, domain
                        2^20, built by the product's statement builder
  prove_2_16_synthetic  a uniform-witness config-5-shaped R1CS, domain 2^16
  prove_2_22_config5    config 5 at its full 2^22 constraints
the 2^22 NTT of config 2, the G1 MSM at config 3's other sizes and with its
witness-like scalars, the G2 MSM of a 2^16 prove, and the CPU oracle's
restatement of the reference algorithms (MSM, NTT, prove) on the host cores,
on one thread and on all the process may use (cpu_baseline), each output
compared with the GPU's.  Prints one JSON line.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
import argparse
import json
import os
import shutil
import sys
import tempfile
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
MADS_PER_FIELD_MUL = 136  # 8x32-bit CIOS Montgomery product: 2*8^2 + 8 word multiply-adds


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def msm_algorithmic_mults(n, c):
    """Algorithmic field multiplications of a G1 MSM of n points with c-bit
    signed windows (W = ceil(255/c)): 10 per mixed addition of every point in
    every window, 14 per bucket-reduction addition (2 per bucket), and 6c + 14
    per window for the window combination."""
    w = -(-255 // c)
    return n * w * 10 + w * (1 << (c - 1)) * 2 * 14 + w * (6 * c + 14)


def best_c(n):
    return min(range(8, 22), key=lambda c: msm_algorithmic_mults(n, c))


def host_cpu():
    """What the process runs on: logical CPUs it may use, the machine's
    logical CPU and socket counts and the CPU model (from /proc/cpuinfo)."""
    info = {"usable_cpus": len(os.sched_getaffinity(0)), "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}
    try:
        txt = open("/proc/cpuinfo").read()
        info["logical_cpus"] = txt.count("processor\t:")
        info["sockets"] = len({l.split(":")[1].strip() for l in txt.splitlines() if l.startswith("physical id")})
        info["model"] = next((l.split(":", 1)[1].strip() for l in txt.splitlines() if l.startswith("model name")), None)
    except OSError:
        pass
    try:  # lscpu's identification lines, as printed
        import subprocess
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        keep = ("Model name", "Vendor ID", "CPU family", "Model", "Stepping", "Thread(s) per core",
                "Core(s) per socket", "Socket(s)", "CPU max MHz", "L3 cache", "Hypervisor vendor")
        info["lscpu"] = {k.strip(): v.strip() for k, v in (l.split(":", 1) for l in out.splitlines() if ":" in l)
                         if k.strip() in keep}
    except (OSError, ValueError, subprocess.SubprocessError):
        pass
    return info


def mont_words(vals):
    """v 2^256 mod r for Python ints v, as (k, 4) uint64 words (Montgomery form)."""
    b = b"".join(((v << 256) % R_ORDER).to_bytes(32, "little") for v in vals)
    return np.frombuffer(b, dtype=np.uint64).reshape(-1, 4).copy()


def witness_like_scalars(n, rng, uniform):
    """BASELINE config 3 (ii): 70% in [0, 2^16), 10% r - [1, 2^16), 20%
    uniform, in Montgomery form (uniform words below r are valid as they are)."""
    small = mont_words(range(1 << 16))
    neg = mont_words([R_ORDER - v for v in range(1 << 16)])
    s = uniform.copy()
    u = rng.random(n)
    m = u < 0.7
    s[m] = small[rng.integers(0, 1 << 16, size=int(m.sum()))]
    m = (u >= 0.7) & (u < 0.8)
    s[m] = neg[rng.integers(1, 1 << 16, size=int(m.sum()))]
    return s


def ntt_case(ctx, ln, rng):
    """Forward NTT of 2^ln uniform Fr elements (config 2): pass-kernel time from
    HIP events, wall time per transform, HBM and VALU fractions.  Returns the
    figures, the input and the output (for the CPU baseline's check)."""
    import zkml_amd
    a = zkml_amd.random_fr(1 << ln, rng)
    da = ctx.upload(a)
    do = ctx.alloc((1 << ln) * 32)
    ctx.ntt(do, da, ln)
    ctx.sync()
    ctx.set_profiling(True, only="ntt_pass")
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
    log(f"[bench] NTT 2^{ln}: {kms:.3f} ms")
    out = ctx.d2h(do, (1 << ln, 4))
    del da, do
    return ntt, a, out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--log-n", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prove", action="store_true")
    ap.add_argument("--msm-only", action="store_true",
                    help="only the 2^20 G1 MSM steps (the run the rocprofv3 counter summaries profile)")
    ap.add_argument("--ntt-only", action="store_true",
                    help="only the forward NTT of 2^22 elements (config 2; the run the NTT counter summaries profile)")
    ap.add_argument("--prove-only", action="store_true",
                    help="only the config 4 (2^16) proves, --steps of them after 3 warm-up proves (the run the "
                         "proof timeline summary traces)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device copy of MIB MiB (torch's copy kernel), the reference for "
                         "scaling rocprofv3 FETCH_SIZE / WRITE_SIZE readings to bytes")
    ap.add_argument("--gather-calibration", type=int, default=0, metavar="MIB",
                    help="only run a gather of random 64-byte rows from an MIB MiB table (torch index_select): "
                         "the reference for scaling FETCH_SIZE of kernels that gather 64-byte point records")
    args = ap.parse_args()
    if args.gather_calibration:
        import torch
        rows = (args.gather_calibration << 20) // 64
        table = torch.ones((rows, 16), dtype=torch.int32, device="cuda")
        idx = torch.randperm(rows, device="cuda")
        for _ in range(3):
            out = table.index_select(0, idx)
        torch.cuda.synchronize()
        print(json.dumps({"rows": rows, "row_bytes_read": 64, "index_bytes_read": 8, "bytes_written": rows * 64,
                          "launches": 3, "sum": int(out[0, 0].item())}), flush=True)
        return
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
    if args.ntt_only:
        ntt, _, _ = ntt_case(ctx, 22, rng)
        print(json.dumps({"ntt_2_22": ntt}), flush=True)
        return
    if args.prove_only:
        from statements import load as load_statement
        nc, nv, npub, _, A, B, C, w = load_statement("config4")
        r = ctx.r1cs(nc, nv, npub, A, B, C)
        with tempfile.TemporaryDirectory() as td:
            ctx.setup(r, 0xDEADBEEF42, os.path.join(td, "pk.bin"), os.path.join(td, "vk.bin"))
            pk = ctx.load_pk(os.path.join(td, "pk.bin"))
            for _ in range(3):
                ctx.prove(pk, r, w, npub, 0xCAFEBABE)
            times = []
            for _ in range(args.steps):
                t0 = time.perf_counter()
                ctx.prove(pk, r, w, npub, 0xCAFEBABE)
                times.append((time.perf_counter() - t0) * 1e3)
            pk.close()
        r.close()
        print(json.dumps({"prove_2_16_config4": {"ms": round(float(np.median(times)), 3),
                                                 "min_ms": round(min(times), 3), "proves": args.steps}}), flush=True)
        return
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
    # timed region: HIP events bracket only the dominant kernel (each timed
    # launch adds two event records to the stream)
    ctx.set_profiling(True, only="msm_accumulate")
    ctx.reset_kernel_stats()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        res = ctx.msm_g1(dp, ds, n)
    ctx.sync()
    t1 = time.perf_counter()
    ms_step = (t1 - t0) * 1e3 / args.steps
    cnt, ms = ctx.kernel_stats("msm_accumulate")
    acc_stat = {"ms_per_step": ms / args.steps, "launches_per_step": cnt / args.steps}
    # per-kernel breakdown from a separate, untimed pass with every kernel bracketed
    prof_steps = 5
    ctx.set_profiling(True)
    ctx.reset_kernel_stats()
    for _ in range(prof_steps):
        ctx.msm_g1(dp, ds, n)
    ctx.sync()
    kernels = {}
    for name in ctx.kernel_names():
        cnt, ms = ctx.kernel_stats(name)
        kernels[name] = {"ms_per_step": ms / prof_steps, "launches_per_step": cnt / prof_steps}
    ctx.set_profiling(False)
    mpoints = n / (ms_step * 1e-3) / 1e6
    log(f"[bench] MSM 2^{args.log_n}: {ms_step:.3f} ms/step, {mpoints:.1f} Mpoints/s")

    # roofline of the dominant kernel (bucket accumulation): every sorted
    # (window, point) entry costs one mixed XYZZ addition = 10 field mults.
    c, windows = zkml_amd.Context.msm_config(n)
    acc_ms = acc_stat["ms_per_step"] / max(acc_stat["launches_per_step"], 1)
    acc_mads = n * windows * 10 * MADS_PER_FIELD_MUL
    achieved = acc_mads / (acc_ms * 1e-3) / 1e12
    # HBM bytes per launch of the same kernel, from the committed rocprofv3
    # FETCH_SIZE / WRITE_SIZE runs (profiles/msm_2e20_pmc_traffic.md), scaled by
    # the counters' reading for a plain copy of known size
    traffic = pmc = None
    tpath = os.path.join(ROOT, "profiles", "msm_2e20_pmc_traffic.json")
    if args.log_n == 20 and os.path.exists(tpath):
        prof = json.load(open(tpath))
        traffic = prof.get("msm_accumulate_bytes_per_launch")
        # issue counters of the same kernel from the committed rocprofv3 run
        # (a separate process: counters are not collected here)
        pmc = {k_: prof.get(k_) for k_ in ("sq_insts_valu_per_launch", "sq_active_inst_valu_per_launch", "valu_busy",
                                            "clock_ghz", "lane_instructions_per_mixed_add")}
        pmc["source"] = "profiles/msm_2e20_pmc_traffic.md"
    # whole-MSM VALU fraction from the algorithmic multiplication count above
    f_mults = msm_algorithmic_mults(n, best_c(n))
    msm_frac = f_mults * MADS_PER_FIELD_MUL / (ms_step * 1e-3) / 1e12 / PEAK_MAD_TOPS

    # ---------------- G1 MSM at config 3's other sizes and scalar mix, G2 at 2^16
    def time_msm(fn, d_pts, d_sc, count, reps):
        fn(d_pts, d_sc, count)
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(reps):
            fn(d_pts, d_sc, count)
        ctx.sync()
        return (time.perf_counter() - t0) * 1e3 / reps

    def msm_entry(ms, count, g2=False):
        mults = msm_algorithmic_mults(count, best_c(count)) * (3 if g2 else 1)  # Fp2 mult = 3 Fp mults
        return {"ms": round(ms, 4), "Mpoints_per_s": round(count / (ms * 1e-3) / 1e6, 2),
                "field_mults_per_s": float(f"{mults / (ms * 1e-3):.4g}"),
                "valu_frac": round(mults * MADS_PER_FIELD_MUL / (ms * 1e-3) / 1e12 / PEAK_MAD_TOPS, 4)}

    msm_more = {}
    if args.msm_only:
        args.no_prove = args.no_cpu = True
    else:
        # the same points converted to records once (zk_msm_prepare_points):
        # the per-call conversion is left out of the prepared line only; the
        # per-call line beside it is timed the same way (no per-kernel events)
        msm_more[f"g1_2_{args.log_n}_per_call"] = msm_entry(time_msm(ctx.msm_g1, dp, ds, n, 20), n)
        d_recs = ctx.msm_prepare(dp, n)
        msm_more[f"g1_2_{args.log_n}_prepared"] = msm_entry(time_msm(ctx.msm_g1_prepared, d_recs, ds, n, 20), n)
        del d_recs
        sk = witness_like_scalars(n, rng, s)
        d_sk = ctx.upload(sk)
        msm_more[f"g1_2_{args.log_n}_witness_like"] = msm_entry(time_msm(ctx.msm_g1, dp, d_sk, n, 10), n)
        del d_sk
        for ln_ in (16, 18):
            msm_more[f"g1_2_{ln_}"] = msm_entry(time_msm(ctx.msm_g1, dp, ds, 1 << ln_, 20), 1 << ln_)
        n22 = 1 << 22
        k22 = zkml_amd.random_fr(n22, rng)
        d_k22 = ctx.upload(k22)
        dp22 = ctx.alloc(n22 * 64)
        ctx.g1_generator_mul(d_k22, n22, dp22)
        ds22 = ctx.upload(zkml_amd.random_fr(n22, rng))
        msm_more["g1_2_22"] = msm_entry(time_msm(ctx.msm_g1, dp22, ds22, n22, 5), n22)
        del d_k22, dp22, ds22, k22
        n16 = 1 << 16
        d_k2 = ctx.upload(k[:n16].copy())
        dp2 = ctx.alloc(n16 * 128)
        ctx.g2_generator_mul(d_k2, n16, dp2)
        msm_more["g2_2_16"] = msm_entry(time_msm(ctx.msm_g2, dp2, ds, n16, 20), n16, g2=True)
        del d_k2, dp2
        # G2 at config 5's size (the B query of the 2^22 proof)
        k22 = zkml_amd.random_fr(n22, rng)
        d_k22 = ctx.upload(k22)
        dp22 = ctx.alloc(n22 * 128)
        ctx.g2_generator_mul(d_k22, n22, dp22)
        ds22 = ctx.upload(zkml_amd.random_fr(n22, rng))
        msm_more["g2_2_22"] = msm_entry(time_msm(ctx.msm_g2, dp22, ds22, n22, 5), n22, g2=True)
        del d_k22, dp22, ds22, k22
    for key, v in msm_more.items():
        log(f"[bench] MSM {key}: {v['ms']:.3f} ms, {v['Mpoints_per_s']} Mpoints/s")

    # ---------------- NTT 2^22 (config 2)
    ntt = None
    ln = 22
    if not args.msm_only:
        ntt, ntt_in, ntt_out = ntt_case(ctx, ln, rng)

    # ---------------- full prove at 2^16
    prove = prove_syn = prove22 = prove_c1 = prove_c4n = None
    work = tempfile.TemporaryDirectory()
    kept = {}  # config 4: statement, PK path and GPU proof, for the CPU prove
    if not args.no_prove:
        from statements import load as load_statement

        def prove_case(stmt, reps, label, keep=False):
            """GPU setup, then `reps` proves of a statement (nc, nv, npub, A, B, C,
            w) with the witness handed over from host memory; the proof is
            checked with the product's verifier.  Loading the PK (file read and
            upload) is timed on its own, outside the proves."""
            nc, nv, npub, A, B, C, w = stmt
            log(f"[bench] {label}: {nc} constraints, GPU setup")
            r = ctx.r1cs(nc, nv, npub, A, B, C)
            td = tempfile.mkdtemp(dir=work.name)
            pk_path = os.path.join(td, "pk.bin")
            t0 = time.perf_counter()
            ctx.setup(r, 0xDEADBEEF42, pk_path, os.path.join(td, "vk.bin"))
            t_setup = time.perf_counter() - t0
            t0 = time.perf_counter()
            pk = ctx.load_pk(pk_path)
            t_load = time.perf_counter() - t0
            vk_bytes = open(os.path.join(td, "vk.bin"), "rb").read()
            if not keep:
                shutil.rmtree(td)
            for _ in range(3):  # warm-up (workspaces, streams, host threads)
                ctx.prove(pk, r, w, npub, 0xCAFEBABE)
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
                   "ms": round(float(np.median(times)), 3), "min_ms": round(float(np.min(times)), 3),
                   "setup_s": round(t_setup, 2), "pk_load_s": round(t_load, 3), "proof_verifies": ok,
                   "breakdown_ms": {k_: round(v, 3) for k_, v in parts.items()}}
            log(f"[bench] {label}: {out['ms']:.3f} ms (median of {reps}), setup {t_setup:.1f} s, verifies: {ok}")
            if keep:
                kept.update(stmt=stmt, pk_path=pk_path, proof=proof)
            pk.close()
            r.close()
            return out

        def synthetic(nc, seed):
            A, B, C, w = zkml_amd.synthetic_r1cs(nc, 4, 16, seed)
            return nc, w.shape[0], 4, A, B, C, w

        def fixture(name):
            nc, nv, npub, npriv, A, B, C, w = load_statement(name)
            if name == "config4":
                kept["npriv"] = npriv
            return nc, nv, npub, A, B, C, w

        prove = prove_case(fixture("config4"), 41, "prove config 4 (2^16)", keep=True)
        prove_c1 = prove_case(fixture("config1"), 41, "prove config 1 (2^13)")
        import statement_models
        st4 = statement_models.config4_named()
        prove_c4n = prove_case((st4.nc, st4.nv, st4.npub, st4.A, st4.B, st4.C, st4.w), 11,
                               "prove config 4 as named (2^20)")
        del st4
        prove_syn = prove_case(synthetic((1 << 16) - 64, 16), 21, "prove 2^16 synthetic")
        prove22 = prove_case(synthetic(1 << 22, 22), 5, "prove 2^22 (config 5)")

    # ---------------- CPU baseline (oracle restatement of the reference MSM)
    # On one thread (the reference's host code) and on every thread OpenMP may
    # use (windows, butterflies and rows in parallel); each output is compared
    # with the GPU's for the same input.
    cpu = None
    if not args.no_cpu:
        from bindings import OracleR1CS, oracle, ptr
        lib = oracle()
        all_threads = int(lib.orc_threads_max())
        pts = ctx.d2h(dp, (n, 8))
        sc = np.ascontiguousarray(s)
        msm_cpu = {}
        for threads in sorted({1, all_threads}):
            out = np.zeros(8, dtype=np.uint64)
            t0 = time.perf_counter()
            lib.orc_msm_g1(ptr(pts), ptr(sc), n, 0, threads, ptr(out))
            dt = time.perf_counter() - t0
            msm_cpu[threads] = {"s": round(dt, 3), "Mpoints_per_s": round(n / dt / 1e6, 4),
                                "equals_gpu": bool(np.array_equal(out, res))}
            log(f"[bench] CPU MSM 2^{args.log_n}, {threads} threads: {dt:.2f} s, equals GPU: "
                f"{msm_cpu[threads]['equals_gpu']}")
        del pts
        ntt_cpu = {}
        for threads in sorted({1, all_threads}):
            b = np.ascontiguousarray(ntt_in.copy())
            t0 = time.perf_counter()
            lib.orc_ntt(ptr(b), ln, 0, threads)
            dt = time.perf_counter() - t0
            ntt_cpu[threads] = {"ms": round(dt * 1e3, 1), "equals_gpu": bool(np.array_equal(b, ntt_out))}
            log(f"[bench] CPU NTT 2^{ln}, {threads} threads: {dt * 1e3:.0f} ms")
        prove_cpu = None
        if kept:
            nc, nv, npub, A, B, C, w = kept["stmt"]
            oc = OracleR1CS(nc, nv, npub, kept["npriv"], [(M["row"], M["col"], M["value"]) for M in (A, B, C)])
            # G2 as the reference computes it (every G2 operation through affine
            # coordinates, src/curve/g2.cuh:103-146) and as Jacobian formulas
            # (~12x faster for B): same proof bytes either way
            prove_cpu = {"reference_affine_g2": {}, "jacobian_g2": {}}
            for g2_ref in (True, False):
                key = "reference_affine_g2" if g2_ref else "jacobian_g2"
                for threads in sorted({1, all_threads}):
                    t0 = time.perf_counter()
                    rc, proof_o, ms_o = oc.prove(kept["pk_path"], w, 0xCAFEBABE, threads=threads,
                                                 g2_affine_ref=g2_ref)
                    dt = time.perf_counter() - t0
                    prove_cpu[key][str(threads)] = {
                        "ms": round(dt * 1e3, 1), "equals_gpu": rc == 0 and proof_o == kept["proof"],
                        "phases_ms": {k_: round(float(v), 1) for k_, v in zip(("h", "A", "B_g2", "C"), ms_o)}}
                    log(f"[bench] CPU prove config 4 ({key}), {threads} threads: {dt * 1e3:.0f} ms, equals GPU: "
                        f"{prove_cpu[key][str(threads)]['equals_gpu']}")
        top = msm_cpu[all_threads]
        cpu = {"value": top["Mpoints_per_s"], "unit": "Mpoints/s", "cores": all_threads, "kind": "port",
               "sample": f"G1 MSM over the same 2^{args.log_n} points/scalars, reference Pippenger (MSMConfig "
                         f"windows, Jacobian mixed adds, serial running sums; one window per OpenMP thread), "
                         f"{top['s']} s on {all_threads} threads",
               "single_thread": msm_cpu[1], "all_threads": top,
               "ntt_2_22_ms": {"1": ntt_cpu[1], str(all_threads): ntt_cpu[all_threads]},
               "prove_2_16_ms": prove_cpu,
               "host": host_cpu()}
    work.cleanup()

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
        "field_mults_per_s": float(f"{f_mults / (ms_step * 1e-3):.4g}"),
        "field_mults_per_step": f_mults,
        "pmc_msm_accumulate": pmc,
        "msm_more": msm_more,
        "kernels_ms_per_step": {k_: round(v["ms_per_step"], 4) for k_, v in kernels.items()},
        "prove_2_16": prove,
        "prove_2_16_synthetic": prove_syn,
        "prove_config1": prove_c1,
        "prove_config4_named": prove_c4n,
        "prove_2_22_config5": prove22,
        "ntt_2_22": ntt,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
