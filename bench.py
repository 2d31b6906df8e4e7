"""Keyswitch/rotation throughput of the gfx950 RNS-CKKS backend.

Workload (one GPU): 64 ciphertexts at N = 2^16 (2^15 slots, values
uniform[-1, 1] from seed 0), Q = one 60-bit + 35 40-bit primes, dnum 3 hybrid
key switching with 12 44-bit special primes.  One step = rotations by
2^0 .. 2^14 of all 64 ciphertexts (chained, 15 x 64 key switches at 36 limbs),
then HMult + relinearise + rescale at every level 36 -> 2 (34 x 64 key
switches).  Inputs are resident in HBM before the timed region.

Prints one JSON line: keyswitch/s, the roofline of the dominant kernel (the
two-pass NTT, timed with events on the library stream) and the CPU oracle's
keyswitch rate on the host cores.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "easyfhe-llama3-8b_amd"))

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
# HBM bytes moved by one batch NTT transform per algorithmic byte (read + write
# of each limb-polynomial once): two passes, FETCH_SIZE/WRITE_SIZE counter
# runs calibrated against a device copy (profiles/ntt_batch_pmc_traffic.md)
NTT_TRAFFIC_RATIO = 2.02
# HBM bytes of one key-switch step (64 ciphertexts, 15 rotations + 34 HMult
# levels): FETCH_SIZE x 1.999 + WRITE_SIZE x 1.000 summed over the step's
# kernels in rocprofv3 counter runs of bench.py --mode ks-profile
# (profiles/keyswitch_step_traffic.md); "fused" is the default path,
# "separate" the one with CKKS_KEYSWITCH_FUSED=0
KS_STEP_TRAFFIC = {"fused": 790.9e9, "separate": 1942.6e9}
# 12 special primes of 44 bits: P = 2^528 exceeds the largest digit (2^500) and
# every limb but q_0 takes the fp64 modular-arithmetic path of the NTT
PARAMS = dict(log_n=16, depth=35, dnum=3, dcrt_bits=40, first_mod=60, special_bits=44)
ROTATIONS = tuple(1 << k for k in range(15))


def keyswitch_bytes(N: int, limbs: int, alpha: int, digits: int, batch: int, relin: bool) -> float:
    """Algorithmic HBM bytes per key switch: read c0, c1, write 2 limbs-polys
    (relinearisation also reads d2), plus the key streamed once per batch."""
    polys = (5 if relin else 4) * limbs
    return 8.0 * N * (polys + 2.0 * digits * (limbs + alpha) / batch)


def _oracle_timing_library():
    """The oracle's ORC_FAST build (Shoup reductions, the same words as the
    pinned build) compiled for this host with -O3 -march=native when gcc is
    here, else the prebuilt generic x86-64 one."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import tempfile

    import oracle as O

    src = ROOT / "oracle" / "ckks_oracle.c"
    out = Path(tempfile.mkdtemp(prefix="ckks_oracle_")) / "libckks_oracle_native.so"
    cmd = ["gcc", "-O3", "-march=native", "-std=gnu11", "-fPIC", "-fopenmp", "-ffp-contract=off",
           "-DORC_FAST", "-shared", "-o", str(out), str(src), "-lm"]
    try:
        import subprocess

        subprocess.run(cmd, check=True, capture_output=True, timeout=180)
        return O.load(out), "gcc -O3 -march=native -DORC_FAST (built on this host)"
    except Exception:
        return O.load(O.fast_library_path()), "gcc -O3 -DORC_FAST, generic x86-64 (prebuilt)"


def _cpu_threads() -> tuple[int, int, int]:
    """(threads used for the all-core figure, nproc, CPUs in this process's
    affinity mask); a GPU host's share is 16 cores per GPU."""
    nproc = os.cpu_count() or 1
    try:
        aff = len(os.sched_getaffinity(0))
    except AttributeError:
        aff = nproc
    return max(1, min(16, aff)), nproc, aff


def _cpu_rotations(O, lib, threads: int, budget_s: float, cap: int) -> tuple[int, float]:
    """Chained rotations of one full-size ciphertext (36 limbs, N = 2^16,
    dnum 3, 12 special primes) on `threads` threads within about budget_s."""
    lib.orc_set_threads(int(threads))
    L = PARAMS["depth"] + 1
    ctx = O.OracleContext(log_n=16, limbs=L, alpha=12, dnum=3, first_bits=60, dcrt_bits=40,
                          special_bits=PARAMS["special_bits"], seed=0, library=lib)
    g = ctx.galois_elt(1)
    ctx.gen_rotation_key(g)
    z = np.random.default_rng(0).uniform(-1, 1, 1 << 15)
    ct = ctx.encrypt(z, slots=1 << 15, scale=2.0**40, limbs=L, enc_id=1)
    n, t0 = 0, time.perf_counter()
    while True:
        ct = ctx.rotate_g(ct, g)
        n += 1
        if time.perf_counter() - t0 > budget_s or n >= cap:
            break
    dt = time.perf_counter() - t0
    ctx.close()
    return n, dt


def _cpu_matvec(O, lib, threads: int) -> dict:
    """The CPU matvec workload end to end on the oracle: N = 2^13, 4 x 40-bit
    limbs + one 60-bit special prime, W and x uniform[-1, 1] from seed 0, BSGS
    B = 16, G = 8, 32 token lanes; keys, encode and encrypt timed as set-up,
    then the hoisted MAC + rescale + decrypt, checked against fp64 W x."""
    lib.orc_set_threads(int(threads))
    D, lanes, B, G = 128, 32, 16, 8
    t0 = time.perf_counter()
    ctx = O.OracleContext(log_n=13, limbs=4, alpha=1, dnum=4, first_bits=40, dcrt_bits=40,
                          special_bits=60, seed=0, library=lib)
    for o in list(range(lanes, B * lanes, lanes)) + [B * lanes]:
        ctx.gen_rotation_key(ctx.galois_elt(o))
    slots = ctx.N // 2
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    feat = np.arange(slots) // lanes
    rows = [W[(feat - g * B) % D, (feat + b) % D] for g in range(G) for b in range(B)]
    pts = np.stack([ctx.encode(r, slots=slots, scale=2.0**40, limbs=4) for r in rows])
    ct = ctx.encrypt(packed, slots=slots, scale=2.0**40, limbs=4, enc_id=41)
    setup = time.perf_counter() - t0
    t0 = time.perf_counter()
    acc = ctx.hoisted_mac_sum(ct, [ctx.galois_elt(lanes * b) for b in range(B)], pts,
                              ctx.galois_elt(B * lanes), G)
    out = ctx.rescale(acc)
    sc = 2.0**80 / float(ctx.primes[3])
    dec = ctx.decrypt(out, slots=slots, scale=sc).real[np.arange(D) * lanes]
    run = time.perf_counter() - t0
    ctx.close()
    return {"setup_s": round(setup, 4), "matvec_s": round(run, 4),
            "max_abs_err_vs_fp64": float(np.abs(dec - W @ x).max())}


def cpu_baseline(seconds_budget: float = 20.0) -> dict:
    """The oracle (the same algorithms as the kernels) on the host cores: the
    full-size key switch on one thread and on all of this GPU's cores, and the
    N = 2^13 matvec workload end to end."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as O

    lib, build = _oracle_timing_library()
    threads, nproc, aff = _cpu_threads()
    n1, t1 = _cpu_rotations(O, lib, 1, 0.3 * seconds_budget, 8)
    n, t = _cpu_rotations(O, lib, threads, 0.5 * seconds_budget, 64)
    mv1 = _cpu_matvec(O, lib, 1)
    mv = _cpu_matvec(O, lib, threads)
    return {"value": n / t, "unit": "keyswitch/s", "cores": threads, "kind": "port",
            "sample": f"{n} chained rotations of one ciphertext at 36 limbs, N=2^16, dnum 3, "
                      f"12 special primes, on {threads} threads (oracle/ckks_oracle.c, OpenMP "
                      f"over limbs and coefficients); {n1} on one thread",
            "single_thread_value": n1 / t1,
            "build": build, "nproc": nproc, "affinity_cpus": aff,
            "matvec_config": {"workload": "BSGS matvec, N=2^13, 4x40b limbs + 1x60b special, "
                                          "128x128 W, B=16, G=8, seed 0",
                              "one_thread": mv1, f"{threads}_threads": mv}}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--cts", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-bootstrap", action="store_true",
                    help="skip the bootstrap measurement of the default run")
    ap.add_argument("--no-linear", action="store_true",
                    help="skip the feature-major linear measurement of the default run")
    ap.add_argument("--levels", type=int, default=34, help="HMult levels per step")
    ap.add_argument("--no-mlp", action="store_true",
                    help="skip the RMSNorm + MLP block measurement of the default run")
    ap.add_argument("--no-attention", action="store_true",
                    help="skip the attention measurement of the default run")
    ap.add_argument("--no-prefill", action="store_true",
                    help="skip the 32-layer prefill on the reference's chain")
    ap.add_argument("--no-layer", action="store_true",
                    help="skip the refreshed-layer measurement of the default run")
    ap.add_argument("--layers", type=int, default=None,
                    help="layers of the layers mode (default 2) and of the prefill mode "
                         "(default 32)")
    ap.add_argument("--mode", choices=["keyswitch", "ntt-profile", "ks-profile", "int-peak",
                                       "prefill-reference-chain",
                                       "bootstrap", "linear", "mlp", "attention", "layer",
                                       "layers", "layers-reference-chain", "prefill"],
                    default="keyswitch",
                    help="ntt-profile: only the batch NTT and a 36 MiB device copy "
                         "(the calibration kernel), for rocprofv3 counter runs; "
                         "ks-profile: one key-switch step and a 36 MiB device copy, for "
                         "rocprofv3 counter runs; "
                         "int-peak: the register-only integer-throughput probes; "
                         "bootstrap: the full-slot bootstrap workload on the same chain; "
                         "linear: one 4096x4096 feature-major linear over 128 tokens; "
                         "mlp: the RMSNorm + SwiGLU MLP + residual half of a layer; "
                         "attention: the causal attention of a layer; "
                         "layer: one whole encrypted decoder layer on a deeper chain; "
                         "layers: consecutive layers with their bootstraps (--layers); "
                         "layers-reference-chain: the same on the reference's chain "
                         "(60 + 37 x 59-bit primes, dnum 5) with the softmax normalisers "
                         "refreshed; "
                         "prefill: the encrypted prefill from token ids to logits (--layers, "
                         "default 32); prefill-reference-chain: the same on the reference's "
                         "chain and budget (4, 4) with its normaliser and slim RMSNorm "
                         "refreshes")
    ap.add_argument("--boot-cts", type=int, default=32)
    ap.add_argument("--boot-group", type=int, default=16,
                    help="ciphertexts per batched bootstrap group")
    ap.add_argument("--budget", type=int, nargs=2, default=(3, 3))
    ap.add_argument("--linear-strategy", default="normal",
                    choices=["normal", "ext_normal", "ext_double_hoist"],
                    help="hoist strategy of the linear mode")
    ap.add_argument("--linear-rows", type=int, default=512,
                    help="plaintext rows per chunk of the linear mode (512: the reference's "
                         "8 giants of 64 babies)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU; --gpus {args.gpus} is not supported (across GPUs "
              "the key-switch batches and the feature-major ciphertexts would be split by "
              "ciphertext, each GPU holding its own copy of the keys)", file=sys.stderr)
        return 2
    if args.mode in ("prefill", "prefill-reference-chain") or (args.mode == "keyswitch"
                                                               and not args.no_prefill):
        # The plaintext passes run on torch; its bundled HIP runtime must be
        # the process's only one, which holds when torch loads before the
        # backend library (the backend then binds to the runtime by soname).
        import torch  # noqa: F401

    from easyfhe import _native, fhe

    spec = fhe.CKKSContextSpec(depth=PARAMS["depth"], log_n=PARAMS["log_n"], dnum=PARAMS["dnum"],
                               dcrt_bits=PARAMS["dcrt_bits"], first_mod=PARAMS["first_mod"],
                               special_bits=PARAMS["special_bits"], seed=0, rotations=ROTATIONS)
    if args.mode == "ntt-profile":
        return ntt_profile(spec, args.cts)
    if args.mode == "ks-profile":
        return ks_profile(spec, args.cts, args.levels)
    if args.mode == "int-peak":
        spec.rotations = ()
        spec.relin_key = False
        client, ctx = fhe.generate_client_context(spec, device="cuda:0")
        print(json.dumps({"int_peak": int_peaks(ctx)}), flush=True)
        return 0
    if args.mode == "bootstrap":
        return bootstrap_bench(spec, args)
    if args.mode == "linear":
        spec.rotations = ()
        client, ctx = fhe.generate_client_context(spec, device="cuda:0")
        print(json.dumps({"fm_linear": measure_fm_linear(client, ctx, warmup=args.warmup,
                                                         strategy=args.linear_strategy,
                                                         rows=args.linear_rows)}),
              flush=True)
        return 0
    if args.mode == "prefill":
        n = 32 if args.layers is None else args.layers
        print(json.dumps({"fm_prefill": measure_fm_prefill(n)}), flush=True)
        return 0
    if args.mode == "prefill-reference-chain":
        n = 32 if args.layers is None else args.layers
        print(json.dumps({"fm_prefill_reference_chain": measure_fm_prefill(
            n, params=REFERENCE_CHAIN_PARAMS, budget=REFERENCE_BUDGET, refresh_normalisers=True,
            slim_rmsnorm=True)}), flush=True)
        return 0
    if args.mode == "layers":
        print(json.dumps({"fm_layers": measure_fm_layers(2 if args.layers is None
                                                         else args.layers)}), flush=True)
        return 0
    if args.mode == "layers-reference-chain":
        print(json.dumps({"fm_layers_reference_chain": measure_fm_layers(
            2 if args.layers is None else args.layers, params=REFERENCE_CHAIN_PARAMS,
            budget=REFERENCE_BUDGET, refresh_normalisers=True, slim_rmsnorm=True)}), flush=True)
        return 0
    if args.mode == "layer":
        print(json.dumps({"fm_layer": measure_fm_layer(warmup=args.warmup)}), flush=True)
        return 0
    if args.mode == "attention":
        spec.rotations = ()
        client, ctx = fhe.generate_client_context(spec, device="cuda:0")
        print(json.dumps({"fm_attention": measure_fm_attention(client, ctx,
                                                               warmup=args.warmup)}),
              flush=True)
        return 0
    if args.mode == "mlp":
        spec.rotations = ()
        client, ctx = fhe.generate_client_context(spec, device="cuda:0")
        print(json.dumps({"fm_mlp_block": measure_fm_mlp_block(client, ctx,
                                                               warmup=args.warmup)}),
              flush=True)
        return 0
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    ctx.synchronize()
    keygen_s = time.perf_counter() - t0
    N, L, alpha = ctx.N, ctx.L, ctx.alpha
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    cts = [client.encrypt(rng.uniform(-1, 1, slots), slots=slots, enc_id=i + 1)
           for i in range(args.cts)]
    ctx.synchronize()
    levels = min(args.levels, L - 2)

    def step():
        return keyswitch_step(ctx, cts, levels)

    for _ in range(args.warmup):
        out = step()
        for c in out:
            c.release()
    ctx.synchronize()
    ev0 = fhe_event(ctx)
    ev1 = fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
        for c in out:
            c.release()
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    gpu_ms = ev0.elapsed_time(ev1)
    ks_per_step = args.cts * (len(ROTATIONS) + levels)
    ms_per_step = wall * 1000.0 / args.steps
    value = ks_per_step * args.steps / wall

    # algorithmic bytes of the key switches of one step
    digits_at = lambda l: -(-l // ctx.digit_size)  # noqa: E731
    step_bytes = len(ROTATIONS) * args.cts * keyswitch_bytes(N, L, alpha, digits_at(L), args.cts, False)
    for lvl in range(levels):
        l = L - lvl
        step_bytes += args.cts * keyswitch_bytes(N, l, alpha, digits_at(l), args.cts, True)
    ks_gbs = step_bytes * args.steps / wall / 1e9

    # dominant kernel: the two-pass NTT over all limb-polynomials of the batch,
    # timed with events on the library stream (forward then inverse so the
    # data stays valid)
    batch = fhe_ptrs(cts)
    ntt_iters = 5
    e0, e1 = fhe_event(ctx), fhe_event(ctx)
    _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 0))
    _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 1))
    e0.record()
    for _ in range(ntt_iters):
        _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 0))
        _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 1))
    e1.record()
    ctx.synchronize()
    ntt_ms = e0.elapsed_time(e1) / (2 * ntt_iters)  # one full (2-pass) transform of the batch
    limb_polys = len(cts) * 2 * L
    ntt_bytes = limb_polys * 2.0 * 8 * N  # read + write each limb-polynomial once
    achieved = ntt_bytes / (ntt_ms * 1e-3) / 1e9

    result = {
        "metric": "keyswitch/s @N=2^16",
        "value": round(value, 2),
        "unit": "keyswitch/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {
            "workload": "keyswitch/rotation microbench: 64 ciphertexts, N=2^16, Q=1x60b+35x40b, "
                        "dnum=3, P=12x44b; rotations 2^0..2^14 then HMult+relin+rescale 36->2",
            "ciphertexts": args.cts,
            "keyswitches_per_step": ks_per_step,
            "levels_per_step": levels,
        },
        "keyswitch_hbm_gbs": round(ks_gbs, 1),
        "gpu_event_ms_per_step": round(gpu_ms / args.steps, 3),
        "keygen_s": round(keygen_s, 2),
        "roofline": {
            "kernel": "batch NTT (k_ntt16m_* passes, one launch per pass over all limbs: fp64 "
                      "bodies for the 40-bit limbs, the 64-bit body for the 60-bit limb); mean "
                      "of forward and inverse transform",
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": round(ntt_bytes * NTT_TRAFFIC_RATIO),
            "traffic_source": "NTT_TRAFFIC_RATIO from profiles/ntt_batch_pmc_traffic.md",
            "launch_ms": round(ntt_ms, 4),
            "limb_polys_per_launch": limb_polys,
        },
    }
    # one more step with per-kernel timing (events on the library stream,
    # outside the timed region): each kernel group's share of the step, its
    # algorithmic HBM rate and its modular-operation rate against the probes
    peaks = int_peaks(ctx)
    # on one stream, so that the kernels' event windows do not overlap
    ctx.set_split_parts(1)
    ctx.profile(True)
    out = step()
    for c in out:
        c.release()
    prof = ctx.profile_read()
    ctx.profile(False)
    ctx.set_split_parts(0)
    result["int_peak"] = peaks
    result["kernels"] = kernel_table(prof, peaks)
    kernel_bytes = sum(v["bytes"] for v in prof.values())
    path = "separate" if os.environ.get("CKKS_KEYSWITCH_FUSED") == "0" else "fused"
    traffic = KS_STEP_TRAFFIC[path] if args.cts == 64 and levels == 34 else None
    result["keyswitch_roofline"] = {
        "bound": "hbm", "achieved": round(ks_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
        "frac": round(ks_gbs / HBM_PEAK_GBS, 4),
        "algorithmic_bytes_per_step": round(step_bytes),
        "kernel_bytes_per_step": round(kernel_bytes),
        "kernel_over_algorithmic": round(kernel_bytes / step_bytes, 2),
        "path": path,
        "traffic": round(traffic) if traffic else None,
        "traffic_over_algorithmic": round(traffic / step_bytes, 2) if traffic else None,
        "traffic_source": "FETCH_SIZE/WRITE_SIZE counter runs of bench.py --mode ks-profile, "
                          "profiles/keyswitch_step_traffic.md (copied, not measured in this run)",
        "kernels_table": "one extra step on one stream (ckks_set_split_parts(1)), events per "
                         "launch; algorithmic bytes count a squared operand once",
    }
    result["grouped_mac"] = measure_grouped_mac(client, ctx)
    result["matvec_config"] = measure_matvec_config()
    if not (args.no_bootstrap and args.no_linear and args.no_mlp and args.no_attention):
        for c in cts:
            c.release()
    if not args.no_bootstrap:
        # the bootstrap workload on the same chain (32 ciphertexts at one limb)
        result["bootstrap"] = measure_bootstrap(client, ctx, args.boot_cts, args.boot_group,
                                                args.budget, 1)
        # the slim refreshes' shape: 128-slot ciphertexts through the sparse
        # program (sub-sum, then 128-slot transforms)
        result["bootstrap_sparse_128"] = measure_bootstrap(client, ctx, args.boot_cts,
                                                           args.boot_group, args.budget, 1,
                                                           log_slots=7)
    if not args.no_linear:
        # the square linear of a decoder layer on the same chain
        result["fm_linear"] = measure_fm_linear(client, ctx)
    if not args.no_mlp:
        # the RMSNorm + MLP + residual half of a decoder layer on the same chain
        result["fm_mlp_block"] = measure_fm_mlp_block(client, ctx)
    if not args.no_attention:
        # the causal attention of a decoder layer on the same chain
        result["fm_attention"] = measure_fm_attention(client, ctx)
    if not args.no_layer:
        # two whole layers with their bootstraps on the refresh chain (the
        # second in steady state); this chain's keys are freed first
        ctx.close()
        result["fm_layers"] = measure_fm_layers(2)
        # the same layers on the reference's chain (60 + 37 x 59-bit primes,
        # dnum 5), whose bootstraps return fewer levels: every softmax
        # round's normaliser is refreshed as well
        result["fm_layers_reference_chain"] = measure_fm_layers(
            2, params=REFERENCE_CHAIN_PARAMS, budget=REFERENCE_BUDGET, refresh_normalisers=True,
            slim_rmsnorm=True)
    if not args.no_prefill:
        # the 32-layer prefill on the reference's chain and
        # budget, against its ~511 s A100 figure (README.md:9)
        result["fm_prefill_reference_chain"] = measure_fm_prefill(
            32, params=REFERENCE_CHAIN_PARAMS, budget=REFERENCE_BUDGET, refresh_normalisers=True,
            slim_rmsnorm=True)
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline()
    print(json.dumps(result), flush=True)
    return 0


def measure_grouped_mac(client, ctx, limbs: int = 13, reps: int = 20) -> dict:
    """The reference's Q/K gather step (operators/attention/input.py:792-826)
    at N = 2^16: 16 hoisted rotations of one ciphertext kept in Q u P
    (fast_rotate(output_ext=True)), then for each of 4 targets the grouped
    pairwise MAC of its 4 rotations with 4 extended plaintexts (group count
    1, as the reference calls it) and one ModDown.  Times the fused MAC
    (ckks_grouped_mac) against homo_mul_pt + homo_add per term, and reports
    its algorithmic rate (each term's c0, c1 and plaintext word read once,
    each output word written once)."""
    from easyfhe import fhe

    slots = ctx.max_slots
    rng = np.random.default_rng(7)
    ct = client.encrypt(rng.uniform(-1, 1, slots), cur_limbs=limbs, enc_id=880001)
    sc = ct.state.scaling_factor
    offs = [0] + list(ROTATIONS)
    batch = fhe.fast_rotate(ct, offs, ctx, output_ext=True)
    pts = [fhe.encode_rows(ctx, rng.uniform(-1, 1, slots), limbs=limbs, scale=sc, slots=slots,
                           is_ext=True)[0] for _ in offs]
    targets = [(fhe.pack_cipher_batch(batch.cv[4 * t:4 * t + 4]), pts[4 * t:4 * t + 4])
               for t in range(len(offs) // 4)]

    def fused():
        return [fhe.grouped_pairwise_mac(b, p, 1, ctx) for b, p in targets]

    def composed():
        outs = []
        for b, p in targets:
            acc = None
            for c, q in zip(b.cv, p):
                t = fhe.homo_mul_pt(c, q, ctx)
                if acc is None:
                    acc = t
                else:
                    nxt = fhe.homo_add(acc, t, ctx)
                    acc.release()
                    t.release()
                    acc = nxt
            outs.append(acc)
        return outs

    res = {}
    for name, fn in (("fused", fused), ("composed", composed)):
        for c in fn():
            c.release()
        ctx.synchronize()
        ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
        ev0.record()
        for _ in range(reps):
            for c in fn():
                c.release()
        ev1.record()
        ctx.synchronize()
        res[name] = ev0.elapsed_time(ev1) / reps
    E = limbs + ctx.alpha
    terms, groups = len(offs), len(targets)
    alg = 8.0 * ctx.N * E * (3 * terms + 2 * groups)
    for c in batch.cv:
        c.release()
    for b, _ in targets:
        b.release()
    for q in pts:
        q.release()
    ct.release()
    return {"workload": f"{terms} extended hoisted rotations at {limbs} + {ctx.alpha} limbs, "
                        f"N=2^{ctx.logN}, {groups} targets x 4 terms (group count 1 per target)",
            "ms_fused": round(res["fused"], 4), "ms_composed": round(res["composed"], 4),
            "speedup": round(res["composed"] / res["fused"], 2),
            "algorithmic_bytes": round(alg),
            "fused_gbs": round(alg / (res["fused"] * 1e-3) / 1e9, 1),
            "fused_hbm_frac": round(alg / (res["fused"] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def audit_roofline(audit: dict, seconds: float, units: int, unit: str) -> dict:
    """HBM roofline of a whole program from the library's operation audit
    (ckks_audit_read, the analogue of the reference's graph.py:348
    operation_audit): algorithmic bytes = key switches' ciphertext bytes +
    key bytes + plaintext (diagonal) bytes + rescale bytes, over the timed
    wall time, against 8 TB/s."""
    alg = (audit["keyswitch_ct_bytes"] + audit["key_bytes"] + audit["plaintext_bytes"]
           + audit["rescale_bytes"])
    gbs = alg / max(seconds, 1e-9) / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": round(alg),
            f"keyswitches_per_{unit}": round(audit["keyswitches"] / units, 1),
            f"keyswitch_ct_bytes_per_{unit}": round(audit["keyswitch_ct_bytes"] / units),
            f"key_bytes_per_{unit}": round(audit["key_bytes"] / units),
            f"plaintext_bytes_per_{unit}": round(audit["plaintext_bytes"] / units),
            f"rescale_bytes_per_{unit}": round(audit["rescale_bytes"] / units),
            "source": "ckks_audit_read over the timed region"}


def measure_bootstrap(client, ctx, n_cts: int, group: int, budget, warmup: int,
                      log_slots: int | None = None, evalmod=None) -> dict:
    """Bootstrap of n_cts ciphertexts at the bottom level (one limb, values
    uniform[-1, 1] from seed 0) in batched groups: CoeffToSlot / SlotToCoeff
    with the given level budget, EvalMod at a 2^80 working scale,
    output_levels the most the chain allows.  Full-slot by default; with
    log_slots below log N - 1 the sparse program (sub-sum, then the
    2^log_slots-slot transforms) on ciphertexts of that many slots.  Returns
    rate, precision and the program's shape.  `evalmod` (bs.BootstrapParams)
    overrides the program's parameters (linear-level strategy, giants)."""
    import math

    from easyfhe.bs import openfhe as bs

    budget = tuple(int(v) for v in budget)
    ls = ctx.logN - 1 if log_slots is None else int(log_slots)
    probe = bs.BootstrapSpec(log_slots=ls, level_budget=budget, output_levels=0)
    depth = bs.generate(ctx, probe, evalmod).depth_limbs
    bspec = bs.BootstrapSpec(log_slots=ls, level_budget=budget, output_levels=ctx.L - depth - 1)
    t0 = time.perf_counter()
    prog = bs.generate(ctx, bspec, evalmod)
    ctx.synchronize()
    setup_s = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    zs = [rng.uniform(-1, 1, 1 << ls) for _ in range(n_cts)]
    cts = [client.encrypt(z, slots=1 << ls, cur_limbs=1, enc_id=100000 + i)
           for i, z in enumerate(zs)]
    group = max(1, min(group, len(cts)))
    t0 = time.perf_counter()
    for _ in range(max(1, warmup)):
        for o in bs.bootstrap_many(cts[:group], ctx, prog, group=group):
            o.release()
    ctx.synchronize()
    first_s = time.perf_counter() - t0
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ctx.audit(reset=True)
    ev0.record()
    t0 = time.perf_counter()
    outs = bs.bootstrap_many(cts, ctx, prog, group=group)
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    roof = audit_roofline(ctx.audit(reset=True), wall, len(cts), "bootstrap")
    bits = [-math.log2(np.abs(client.decrypt_complex(o) - z).max()) for o, z in zip(outs, zs)]
    for o in outs:
        o.release()
    prog.release()
    return {
        "value": round(len(cts) / wall, 3),
        "unit": "bootstrap/s",
        "ms_per_bootstrap": round(wall * 1000.0 / len(cts), 3),
        "gpu_event_ms_per_bootstrap": round(ev0.elapsed_time(ev1) / len(cts), 3),
        "ciphertexts": len(cts),
        "slots": 1 << ls,
        "subsum_rotations": len(prog.subsum),
        "evalmods_per_ciphertext": 1 if prog.packed else 2,
        "group": group,
        "budget": list(budget),
        "linear_levels": prog.evalmod.strategy,
        "raise_limbs": prog.raise_limbs,
        "output_limbs": prog.output_limbs,
        "evalmod": {"K": prog.evalmod.K, "double_angles": prog.evalmod.double_angles,
                    "degree": len(prog.coefficients) - 1, "depth": prog.cheb_depth,
                    "primes_per_level": prog.step},
        "precision_bits_min": round(min(bits), 2),
        "precision_bits_mean": round(float(np.mean(bits)), 2),
        "setup_s": round(setup_s, 2),
        "first_group_s": round(first_s, 3),
        "roofline": roof,
    }


def measure_fm_linear(client, ctx, limbs: int = 13, warmup: int = 1,
                      strategy: str = "normal", rows: int = 512) -> dict:
    """One 4096 x 4096 feature-major linear (the square projection of a
    Llama-3-8B decoder layer) over 128 tokens = 16 ciphertexts of 8 token
    lanes, entering at `limbs` limbs (the 13-limb QKV budget): the
    reference's production schedule (B = 64, 8 chunks of 8 giants; hoist
    strategy `strategy`, the reference's production one is "normal"), weights
    N(0, 0.02), activations N(0, 1), seed 0.  Timed from the inputs to the
    rescaled outputs, baby rotations included, without synchronisations
    inside the operator (as the layers run it); the per-stage seconds come
    from one more run that synchronises after every stage."""
    from dataclasses import replace

    from feature_major import (FeatureMajorPrefillLayout, LinearOperator, LinearOperatorConfig,
                               LinearWeight, linear_rotations)

    D, lanes = 4096, ctx.max_slots // 4096
    cfg = LinearOperatorConfig(hoist_strategy=strategy, max_plaintext_rows=rows,
                               timed_stages=False)
    t0 = time.perf_counter()
    ctx.generate_rotation_keys(linear_rotations(dimension=D, token_lanes=lanes,
                                                operator_config=cfg))
    ctx.synchronize()
    keygen_s = time.perf_counter() - t0
    lay = FeatureMajorPrefillLayout(seq_len=128, hidden_dim=D, slots=ctx.max_slots)
    rng = np.random.default_rng(0)
    W = rng.normal(0.0, 0.02, (D, D))
    X = rng.normal(0.0, 1.0, (lay.seq_len, D))
    packed = lay.pack(X)
    cts = [client.encrypt(packed[i], cur_limbs=limbs, enc_id=200000 + i)
           for i in range(lay.cipher_count)]
    weight = LinearWeight(W, context=ctx)
    op = LinearOperator(context=ctx, token_lanes=lanes, config=cfg)
    for _ in range(max(1, warmup)):
        outs, _ = op.apply(cts, weight)
        for o in outs:
            o.release()
        op.clear_baby_cache()
    ctx.synchronize()
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    outs, _ = op.apply(cts, weight)
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    op.clear_baby_cache()
    staged = LinearOperator(context=ctx, token_lanes=lanes,
                            config=replace(cfg, timed_stages=True))
    t1 = time.perf_counter()
    souts, profile = staged.apply(cts, weight)
    staged_wall = time.perf_counter() - t1
    for o in souts:
        o.release()
    staged.close()
    plan = op.plan(D)
    per_ct = (len(plan.baby_offsets) - 1 + sum(c.giant_count - 1 for c in plan.chunks)
              + sum(1 for c in plan.chunks if c.giant_base))
    got = lay.unpack(np.stack([client.decrypt(o) for o in outs]))
    err = float(np.abs(got - X @ W.T).max())
    for o in outs:
        o.release()
    op.close()
    weight.close()
    return {
        "seconds": round(wall, 4),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 4),
        "workload": f"4096x4096 feature-major linear, 128 tokens in {len(cts)} ciphertexts of "
                    f"{lanes} lanes at {limbs} limbs; B={plan.baby_steps}, "
                    f"{len(plan.chunks)} chunks of {plan.chunk_giants} giants, hoist strategy "
                    f"{strategy}",
        "keyswitches": per_ct * len(cts),
        "pt_ct_products": D * len(cts),
        "max_abs_err_vs_fp64": err,
        "stages_s": {k: round(v, 4) for k, v in profile.items()},
        "seconds_with_stage_synchronisations": round(staged_wall, 4),
        "rotation_keygen_s": round(keygen_s, 2),
    }


def measure_fm_mlp_block(client, ctx, limbs: int = 20, warmup: int = 1) -> dict:
    """The post-attention half of a Llama-3-8B decoder layer over 128 tokens
    (16 feature-major ciphertexts of 8 lanes): RMSNorm (rsqrt series of
    degree 31 on [0.25, 4]), the SwiGLU MLP (gate/up 14336 x 4096, down
    4096 x 14336, four pages, SiLU series of degree 63 on [-12, 12]) and the
    residual addition, entering at `limbs` limbs.  Weights N(0, 0.02),
    residual stream N(0, 1), seed 0.  The error is against the same
    composition evaluated in fp64 on the plaintexts."""
    from easyfhe.chebyshev import evaluate_direct
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.mlp import FeatureMajorMLPLayout, MLPWeights, mlp_fhe, mlp_rotations
    from feature_major.rmsnorm import residual_add, rmsnorm_fhe, rmsnorm_rotations

    D, I = 4096, 14336
    lay = FeatureMajorPrefillLayout(seq_len=128, hidden_dim=D, slots=ctx.max_slots)
    t0 = time.perf_counter()
    ctx.generate_rotation_keys(sorted(set(rmsnorm_rotations(lay)) | set(mlp_rotations(lay))))
    ctx.synchronize()
    keygen_s = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    G = rng.normal(0.0, 0.02, (I, D))
    U = rng.normal(0.0, 0.02, (I, D))
    Dn = rng.normal(0.0, 0.02, (D, I))
    X = rng.normal(0.0, 1.0, (lay.seq_len, D))
    rs, silu = rsqrt_entry(0.25, 4.0, 31), silu_entry(-12.0, 12.0, 63)
    packed = lay.pack(X)
    cts = [client.encrypt(packed[i], cur_limbs=limbs, enc_id=300000 + i)
           for i in range(lay.cipher_count)]
    mlay = FeatureMajorMLPLayout(lay, I)
    t0 = time.perf_counter()
    weights = MLPWeights(G, U, Dn, silu=silu, layout=mlay, context=ctx)
    ctx.synchronize()
    upload_s = time.perf_counter() - t0

    def run():
        t = {}
        s0 = time.perf_counter()
        norm = rmsnorm_fhe(cts, np.zeros(1), coeffs=rs, layout=lay, crypto_context=ctx)
        t["rmsnorm"] = time.perf_counter() - s0
        s0 = time.perf_counter()
        mlp = mlp_fhe(norm.ciphers, weights, silu=silu, crypto_context=ctx)
        norm.release()
        t["mlp"] = time.perf_counter() - s0
        s0 = time.perf_counter()
        out = residual_add(cts, mlp.ciphers, crypto_context=ctx)
        ctx.synchronize()
        t["residual"] = time.perf_counter() - s0
        stages = dict(mlp.stage_seconds)
        mlp.release()
        return out, t, stages

    for _ in range(max(1, warmup)):
        out, _, _ = run()
        for o in out:
            o.release()
    ctx.synchronize()
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    out, parts, stages = run()
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    got = lay.unpack(np.stack([client.decrypt(o) for o in out]))
    limbs_out = int(out[0].state.cur_limbs)
    for o in out:
        o.release()
    weights.close()
    var = np.mean(X * X, axis=-1, keepdims=True)
    xn = X * evaluate_direct(var, rs["coefficients"], *rs["fit_interval"])
    g = xn @ G.T
    want = X + (evaluate_direct(g, silu["coefficients"], *silu["fit_interval"])
                * (xn @ U.T)) @ Dn.T
    return {
        "seconds": round(wall, 4),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 4),
        "workload": "RMSNorm + SwiGLU MLP (4096 -> 14336 -> 4096, 4 pages) + residual, "
                    f"128 tokens in {lay.cipher_count} ciphertexts of {lay.tokens_per_cipher} "
                    f"lanes, {limbs} -> {limbs_out} limbs",
        "parts_s": {k: round(v, 4) for k, v in parts.items()},
        "mlp_stages_s": {k: round(v, 4) for k, v in stages.items()},
        "max_abs_err_vs_fp64": float(np.abs(got - want).max()),
        "rotation_keygen_s": round(keygen_s, 2),
        "weight_upload_s": round(upload_s, 2),
    }


def measure_fm_attention(client, ctx, limbs: int = 34, warmup: int = 1) -> dict:
    """Causal attention of a Llama-3-8B decoder layer over 128 tokens: 32 query
    heads of 128 (key/value heads already repeated for the query groups), in
    16 feature-major ciphertexts of 8 lanes entering at `limbs` limbs;
    QK, the Algorithm-2 softmax (2 rounds, scores assumed in [-4, 4]) and PV.
    Q, K, V entries N(0, 0.5^2) / N(0, 1), seed 0; the error is against exact
    causal softmax attention in fp64."""
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.attention import (AttentionGeometry, SoftmaxConfig, attention_fhe,
                                         attention_rotations)

    T, D, H, hd = 128, 4096, 32, 128
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=ctx.max_slots)
    geo = AttentionGeometry(lay, H, hd)
    t0 = time.perf_counter()
    ctx.generate_rotation_keys(attention_rotations(geo))
    ctx.synchronize()
    keygen_s = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    q = rng.normal(0, 0.5, (T, D))
    k = rng.normal(0, 0.5, (T, D))
    v = rng.normal(0, 1.0, (T, D))
    cfg = SoftmaxConfig(rounds=2, shift=4.0, bound=4.0)

    def enc(x, base):
        p = lay.pack(x)
        return [client.encrypt(p[i], cur_limbs=limbs, enc_id=base + i)
                for i in range(lay.cipher_count)]

    qc, kc, vc = enc(q, 400000), enc(k, 400100), enc(v, 400200)
    for _ in range(max(1, warmup)):
        res = attention_fhe(qc, kc, vc, geo, cfg, crypto_context=ctx)
        res.release()
    ctx.synchronize()
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    res = attention_fhe(qc, kc, vc, geo, cfg, crypto_context=ctx)
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    got = lay.unpack(np.stack([client.decrypt(o) for o in res.ciphers]))
    limbs_out = int(res.ciphers[0].state.cur_limbs)
    res_stages = dict(res.stage_seconds)
    res.release()
    qh, kh, vh = (a.reshape(T, H, hd).transpose(1, 0, 2) for a in (q, k, v))
    s = qh @ kh.transpose(0, 2, 1) / np.sqrt(hd)
    valid = np.tril(np.ones((T, T), dtype=bool))[None]
    e = np.where(valid, np.exp(np.where(valid, s, 0) - 4.0), 0.0)
    want = ((e / e.sum(-1, keepdims=True)) @ vh).transpose(1, 0, 2).reshape(T, D)
    return {
        "seconds": round(wall, 4),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 4),
        "workload": f"causal attention, 128 tokens x 32 heads x 128 in {lay.cipher_count} "
                    f"ciphertexts of {lay.tokens_per_cipher} lanes, {limbs} -> {limbs_out} limbs; "
                    "Algorithm-2 softmax, 2 rounds",
        "stages_s": {k2: round(v2, 4) for k2, v2 in res_stages.items()},
        "max_abs_err_vs_exact_fp64": float(np.abs(got - want).max()),
        "score_abs_max": float(np.abs(np.where(valid, s, 0)).max()),
        "rotation_keygen_s": round(keygen_s, 2),
        "rotation_keys": len(attention_rotations(geo)),
    }


# A chain that holds one whole decoder layer without a refresh: 60-bit q_0 +
# 72 x 40-bit primes, dnum 5 (digits of 15 primes), 15 special primes of 44
# bits.  (dnum 7, digits of 11 for the tile-resident conversion, measured
# slower here: 7.39 -> 7.98 s, the hoisted rotations' extra digits outweigh it)
LAYER_PARAMS = dict(log_n=16, depth=72, dnum=5, dcrt_bits=40, first_mod=60, special_bits=44)


def randomized_hadamard(dim: int, seed: int) -> np.ndarray:
    """Orthogonal ``H diag(s) / sqrt(dim)`` (Sylvester Hadamard, seeded random
    signs): the QuaRot-style rotation of the residual basis."""
    h = np.ones((1, 1))
    while h.shape[0] < dim:
        h = np.block([[h, h], [h, -h]])
    s = np.random.default_rng(seed).choice([-1.0, 1.0], dim)
    return h * s[None, :] / np.sqrt(dim)


def _memory_summary(mem: dict) -> dict:
    """Pool figures in GiB (byte counts) beside the allocation count."""
    return {(k[:-6] + "_gib" if k.endswith("_bytes") else k):
            (round(v / 2 ** 30, 1) if k.endswith("_bytes") else v) for k, v in mem.items()}


def _layer_weights(rng, D, KV, hd, I, R):
    """Weights N(0, 0.02) in a residual basis rotated by R (QuaRot-style)."""
    return dict(q=rng.normal(0, 0.02, (D, D)) @ R, k=rng.normal(0, 0.02, (KV * hd, D)) @ R,
                v=rng.normal(0, 0.02, (KV * hd, D)) @ R, o=R.T @ rng.normal(0, 0.02, (D, D)),
                gate=rng.normal(0, 0.02, (I, D)) @ R, up=rng.normal(0, 0.02, (I, D)) @ R,
                down=R.T @ rng.normal(0, 0.02, (D, I)))


def _layer_fp64(x, w, ap, H, KV, hd):
    """The layer in fp64 with the fitted RMSNorm / SiLU series and exact
    causal softmax (the plaintext layer the encrypted one approximates)."""
    from easyfhe.chebyshev import evaluate_direct
    from feature_major.rope import rope_angles

    T, D = x.shape

    def rms(a, e):
        var = np.mean(a * a, axis=-1, keepdims=True)
        return a * evaluate_direct(var, e["coefficients"], *e["fit_interval"])

    def rope(a):
        ang = rope_angles(np.arange(T), hd)
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        h = a.reshape(T, H, hd)
        lo, hi = h[..., :hd // 2], h[..., hd // 2:]
        return np.concatenate([lo * c - hi * s, hi * c + lo * s], -1).reshape(T, -1)

    rep = lambda m: np.repeat(m.reshape(KV, hd, -1), H // KV, axis=0).reshape(H * hd, -1)  # noqa: E731
    n1 = rms(x, ap.input_norm)
    q, k, v = rope(n1 @ w["q"].T), rope(n1 @ rep(w["k"]).T), n1 @ rep(w["v"]).T
    qh, kh, vh = (a.reshape(T, H, hd).transpose(1, 0, 2) for a in (q, k, v))
    sc = qh @ kh.transpose(0, 2, 1) / np.sqrt(hd)
    valid = np.tril(np.ones((T, T), dtype=bool))[None]
    m = np.where(valid, sc, -np.inf)
    e = np.where(valid, np.exp(m - m.max(-1, keepdims=True)), 0.0)
    att = ((e / e.sum(-1, keepdims=True)) @ vh).transpose(1, 0, 2).reshape(T, D)
    h1 = x + att @ w["o"].T
    n2 = rms(h1, ap.post_attention_norm)
    g = n2 @ w["gate"].T
    act = evaluate_direct(g, ap.silu["coefficients"], *ap.silu["fit_interval"]) * (n2 @ w["up"].T)
    return h1 + act @ w["down"].T, float(np.abs(np.where(valid, sc, 0)).max())


def measure_fm_layer(warmup: int = 0) -> dict:
    """One Llama-3-8B decoder layer over 128 tokens, end to end and encrypted
    (d=4096, 32 query / 8 key-value heads of 128, SwiGLU 14336, RMSNorm),
    on a chain deep enough for the whole layer (LAYER_PARAMS, no refresh).
    Weights N(0, 0.02) in a residual basis rotated by a seeded randomized
    Hadamard, inputs N(0, 1), seed 0; Alg2 softmax with 3 rounds on scores
    in [-8, 8].  The error is against the same layer in fp64 with exact
    softmax.  The refreshes a shallower chain would add are measured
    separately (`bootstrap`)."""
    from easyfhe import fhe
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.attention import SoftmaxConfig
    from feature_major.layer import (DecoderLayerWeights, LayerApproximations,
                                     decoder_layer_depth, decoder_layer_fhe,
                                     decoder_layer_rotations)

    T, D, H, KV, hd, I = 128, 4096, 32, 8, 128, 14336
    ap = LayerApproximations(rsqrt_entry(0.25, 4.0, 31), rsqrt_entry(0.25, 4.0, 31),
                             silu_entry(-12.0, 12.0, 63),
                             SoftmaxConfig(rounds=3, shift=8.0, bound=8.0, exp_degree=9,
                                           first_inverse_degree=31, inverse_degree=47))
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=32768)
    spec = fhe.CKKSContextSpec(**LAYER_PARAMS, seed=0,
                               rotations=decoder_layer_rotations(lay, H, hd))
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    ctx.synchronize()
    keygen_s = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    wm = _layer_weights(rng, D, KV, hd, I, randomized_hadamard(D, 1))
    x = rng.normal(0, 1, (T, D))
    packed = lay.pack(x)
    xc = [client.encrypt(packed[i], enc_id=500000 + i) for i in range(lay.cipher_count)]
    t0 = time.perf_counter()
    w = DecoderLayerWeights(wm["q"], wm["k"], wm["v"], wm["o"], wm["gate"], wm["up"], wm["down"],
                            heads=H, kv_heads=KV, head_dim=hd,
                            intermediate=I, approx=ap, layout=lay, context=ctx)
    ctx.synchronize()
    upload_s = time.perf_counter() - t0
    for _ in range(max(0, warmup)):
        decoder_layer_fhe(xc, w, crypto_context=ctx).release()
    ctx.synchronize()
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    res = decoder_layer_fhe(xc, w, crypto_context=ctx)
    ev1.record()
    ctx.synchronize()
    wall = time.perf_counter() - t0
    got = lay.unpack(np.stack([client.decrypt(o) for o in res.ciphers]))
    limbs_out = res.output_limbs
    stages = dict(res.stage_seconds)
    res.release()
    w.close()
    mem = ctx.memory_info()
    ctx.close()

    want, score_max = _layer_fp64(x, wm, ap, H, KV, hd)
    return {
        "seconds": round(wall, 3),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 3),
        "workload": "one Llama-3-8B decoder layer (d=4096, 32/8 heads x 128, SwiGLU 14336), "
                    "128 tokens in 16 ciphertexts of 8 lanes, N=2^16, Q=1x60b+72x40b, dnum=5, "
                    f"P=15x44b; {ctx.L} -> {limbs_out} limbs, no refresh "
                    f"(depth {decoder_layer_depth(ap, T)})",
        "stages_s": {k2: round(v2, 3) for k2, v2 in stages.items()},
        "max_abs_err_vs_fp64": float(np.abs(got - want).max()),
        "output_abs_max": float(np.abs(want).max()),
        "score_abs_max": score_max,
        "rotation_keys": len(spec.rotations),
        "keygen_s": round(keygen_s, 2),
        "weight_upload_s": round(upload_s, 2),
        "device_memory": _memory_summary(mem),
    }


# A chain for refreshed layers: bootstraps (budget (3,3), 26 limbs) return the
# 40 limbs of a layer's deepest block (scores -> softmax -> PV -> W_o).  dnum 6
# keeps digits of 11 limbs and 11 special primes (P = 2^484 above the largest
# digit, 60 + 10 x 40 bits), within the tile-resident conversion's three
# source quads: 2.95 -> 2.69 s per layer against dnum 5, and a smaller P
REFRESH_PARAMS = dict(log_n=16, depth=65, dnum=6, dcrt_bits=40, first_mod=60, special_bits=44)
# the reference's layer chain (assets/feature_major.json:3-16): 60 + 37 x 59-bit
# primes, dnum 5; 8 special primes of 60 bits (P = 2^480 exceeds the largest
# digit, 60 + 7 x 59 = 473 bits)
REFERENCE_CHAIN_PARAMS = dict(log_n=16, depth=37, dnum=5, dcrt_bits=59, first_mod=60,
                              special_bits=60)


# the reference's CoeffToSlot / SlotToCoeff level budget (schedule.py
# bootstrap_level_budget, assets/feature_major.json)
REFERENCE_BUDGET = (4, 4)


def measure_fm_layers(n_layers: int = 2, weight_sets: int = 2, *, params=None,
                      budget=(3, 3), refresh_normalisers: bool = False,
                      slim_rmsnorm: bool = False) -> dict:
    """Consecutive Llama-3-8B decoder layers over 128 tokens with their
    refreshes (bootstraps included): per layer, paired batched refreshes of
    the residual stream before each RMSNorm and of the softmax's mapped
    scores (24 ciphertext bootstraps), on REFRESH_PARAMS (or `params`) with
    CoeffToSlot / SlotToCoeff budget `budget`.  With `refresh_normalisers`
    every softmax round's slim normaliser is bootstrapped too (3 more
    bootstraps per layer), which lets the layer run on a chain whose
    bootstraps return fewer levels (the reference's); with `slim_rmsnorm` the
    post-attention RMSNorm refreshes its slim series (one more bootstrap per
    layer), which lets the residual refreshes return fewer levels (the
    reference's budget (4, 4) on its chain).  The first layer
    starts from a one-limb input; from the second on a layer runs in steady
    state.  Weights N(0, 0.02) in a Hadamard-rotated residual basis,
    `weight_sets` distinct sets cycled over the layers; inputs N(0, 1); seed
    0.  The error is against the same layers in fp64 with exact softmax."""
    from easyfhe import fhe
    from feature_major import FeatureMajorPrefillLayout
    from feature_major.approx import rsqrt_entry, silu_entry
    from feature_major.attention import SoftmaxConfig
    from feature_major.layer import (DecoderLayerWeights, LayerApproximations,
                                     decoder_layer_refreshed_fhe, decoder_layer_rotations,
                                     normaliser_program, refreshed_layer_programs,
                                     rmsnorm_slim_program)

    params = REFRESH_PARAMS if params is None else params
    T, D, H, KV, hd, I = 128, 4096, 32, 8, 128, 14336
    norm = rsqrt_entry(0.5, 16.0, 63)
    ap = LayerApproximations(norm, norm, silu_entry(-12.0, 12.0, 63),
                             SoftmaxConfig(rounds=3, shift=10.0, bound=10.0, exp_degree=7,
                                           first_inverse_degree=31, inverse_degree=47))
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=32768)
    spec = fhe.CKKSContextSpec(**params, seed=0, rotations=decoder_layer_rotations(lay, H, hd))
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    prog, res_prog = refreshed_layer_programs(ctx, ap, T, log_slots=15, level_budget=budget,
                                              refresh_normalisers=refresh_normalisers,
                                              slim_rmsnorm=slim_rmsnorm)
    lam_prog = (normaliser_program(ctx, ap, T, log_slots=15, level_budget=budget)
                if refresh_normalisers else None)
    rms_prog = (rmsnorm_slim_program(ctx, ap, T, log_slots=15, level_budget=budget,
                                     refresh_normalisers=refresh_normalisers)
                if slim_rmsnorm else None)
    ctx.synchronize()
    setup_s = time.perf_counter() - t0
    rng = np.random.default_rng(0)
    R = randomized_hadamard(D, 1)
    wsets = [_layer_weights(rng, D, KV, hd, I, R) for _ in range(max(1, weight_sets))]
    x = rng.normal(0, 1, (T, D))
    t0 = time.perf_counter()
    dev = [DecoderLayerWeights(w["q"], w["k"], w["v"], w["o"], w["gate"], w["up"], w["down"],
                               heads=H, kv_heads=KV, head_dim=hd, intermediate=I, approx=ap,
                               layout=lay, context=ctx) for w in wsets]
    ctx.synchronize()
    upload_s = time.perf_counter() - t0
    packed = lay.pack(x)
    from easyfhe.bs import openfhe as bs

    # the lowest level a refresh takes on this chain (two limbs when the
    # primes are about as wide as q_0)
    start = bs.input_limbs(ctx)
    cur = [client.encrypt(packed[i], cur_limbs=start, enc_id=600000 + i)
           for i in range(lay.cipher_count)]
    per_layer, stages, audit = [], {}, None
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t_all = time.perf_counter()
    for layer in range(int(n_layers)):
        if layer == min(1, int(n_layers) - 1):
            ctx.synchronize()
            ctx.audit(reset=True)  # the audit covers the steady-state layers
        res = decoder_layer_refreshed_fhe(cur, dev[layer % len(dev)], crypto_context=ctx,
                                          program=prog, residual_program=res_prog,
                                          normaliser_program=lam_prog,
                                          rmsnorm_program=rms_prog)
        for c in cur:
            c.release()
        cur = list(res.ciphers)
        per_layer.append(res.wall_seconds)
        stages = res.stage_seconds
        print(f"layer {layer}: {res.wall_seconds:.2f} s, {cur[0].state.cur_limbs} limbs out",
              file=sys.stderr, flush=True)
    ev1.record()
    ctx.synchronize()
    audit = ctx.audit(reset=True)
    total = time.perf_counter() - t_all
    got = lay.unpack(np.stack([client.decrypt(o) for o in cur]))
    out_limbs = int(cur[0].state.cur_limbs)
    for c in cur:
        c.release()
    for d in dev:
        d.close()
    mem = ctx.memory_info()
    L, alpha, primes = ctx.L, ctx.alpha, [int(q) for q in ctx.primes()]
    ctx.close()
    want, smax = x, 0.0
    for layer in range(int(n_layers)):
        want, s_ = _layer_fp64(want, wsets[layer % len(wsets)], ap, H, KV, hd)
        smax = max(smax, s_)
    steady = per_layer[1:] or per_layer
    return {
        "seconds_per_layer": round(float(np.mean(steady)), 3),
        "roofline": audit_roofline(audit, float(np.sum(steady)), len(steady), "layer"),
        "layers": int(n_layers),
        "total_seconds": round(total, 3),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 3),
        "per_layer_s": [round(v, 3) for v in per_layer],
        "workload": f"{n_layers} Llama-3-8B decoder layers (d=4096, 32/8 heads x 128, SwiGLU 14336) "
                    "over 128 tokens in 16 ciphertexts of 8 lanes, bootstraps included "
                    "(3 paired refreshes = 24 bootstraps per layer"
                    + (", plus 3 softmax normaliser refreshes" if refresh_normalisers else "")
                    + (", plus 1 slim RMSNorm refresh" if slim_rmsnorm else "")
                    + f"), N=2^16, Q=1x{params['first_mod']}b+{L - 1}x{params['dcrt_bits']}b, "
                    f"dnum={params['dnum']}, P={alpha}x{params['special_bits']}b, CtS/StC budget "
                    f"{tuple(budget)}; bootstraps return {prog.output_limbs} limbs (scores) "
                    f"and {res_prog.output_limbs} (residual stream); "
                    f"{len(wsets)} weight sets cycled",
        "log_qp_bits": round(sum(math.log2(q) for q in primes), 1),
        "last_layer_stages_s": {k: round(v, 3) for k, v in stages.items()},
        "max_abs_err_vs_fp64": float(np.abs(got - want).max()),
        "output_abs_max": float(np.abs(want).max()),
        "score_abs_max": smax,
        "output_limbs": out_limbs,
        "setup_s": round(setup_s, 2),
        "weight_upload_s": round(upload_s, 2),
        "device_memory": _memory_summary(mem),
    }


def _cheb_torch(x, entry):
    """Chebyshev series of a fitted entry (first coefficient halved) by
    Clenshaw's recurrence, elementwise on a torch tensor."""
    lo, hi = (float(v) for v in entry["fit_interval"])
    c = [float(v) for v in entry["coefficients"]]
    y = (2.0 * x - (lo + hi)) / (hi - lo)
    b1, b2 = x.new_zeros(()), x.new_zeros(())
    for ck in reversed(c[1:]):
        b1, b2 = ck + 2.0 * y * b1 - b2, b1
    return 0.5 * c[0] + y * b1 - b2


class _TorchLayer:
    """A decoder layer in fp64 on the GPU for the prefill's plaintext passes:
    exact (rsqrt, SiLU, softmax) or with the layer's fitted RMSNorm and SiLU
    series (softmax exact)."""

    def __init__(self, w, *, H, KV, hd, T, eps=1e-5, device="cuda"):
        import torch

        from feature_major.rope import rope_angles

        self.w, self.H, self.KV, self.hd, self.eps = w, H, KV, hd, eps
        ang = torch.tensor(rope_angles(np.arange(T), hd), dtype=torch.float64, device=device)
        self.cos, self.sin = torch.cos(ang)[:, None, :], torch.sin(ang)[:, None, :]
        self.mask = torch.tril(torch.ones(T, T, dtype=torch.bool, device=device))

    def _rope(self, a):
        import torch

        T = a.shape[0]
        h = a.reshape(T, -1, self.hd)
        lo, hi = h[..., :self.hd // 2], h[..., self.hd // 2:]
        return torch.cat([lo * self.cos - hi * self.sin, hi * self.cos + lo * self.sin],
                         -1).reshape(T, -1)

    def __call__(self, x, ap=None):
        """(output, h1, gate, scores) for input ``x`` [T, D]."""
        import torch

        w, H, KV, hd = self.w, self.H, self.KV, self.hd
        T = x.shape[0]

        def norm(a, entry):
            ms = (a * a).mean(-1, keepdim=True)
            return a * (torch.rsqrt(ms + self.eps) if entry is None else _cheb_torch(ms, entry))

        n1 = norm(x, None if ap is None else ap.input_norm)
        q = self._rope(n1 @ w["q"].T)
        k = self._rope(n1 @ w["k"].T).reshape(T, KV, hd).repeat_interleave(H // KV, 1)
        v = (n1 @ w["v"].T).reshape(T, KV, hd).repeat_interleave(H // KV, 1)
        qh = q.reshape(T, H, hd).transpose(0, 1).contiguous()
        kt = k.permute(1, 2, 0).contiguous()
        vh = v.transpose(0, 1).contiguous()
        sc = torch.matmul(qh, kt) / float(np.sqrt(hd))
        p = torch.softmax(sc.masked_fill(~self.mask, float("-inf")), -1)
        att = torch.matmul(p, vh).transpose(0, 1).reshape(T, -1)
        h1 = x + att @ w["o"].T
        n2 = norm(h1, None if ap is None else ap.post_attention_norm)
        g = n2 @ w["gate"].T
        act = torch.nn.functional.silu(g) if ap is None else _cheb_torch(g, ap.silu)
        return h1 + (act * (n2 @ w["up"].T)) @ w["down"].T, h1, g, sc


def measure_fm_prefill(n_layers: int = 32, vocab: int = 128256, seed: int = 0, *, params=None,
                       budget=(3, 3), refresh_normalisers: bool = False,
                       slim_rmsnorm: bool = False) -> dict:
    """The full encrypted Llama-3-8B prefill over 128 tokens: random token
    ids (seed) embedded by the client, ``n_layers`` encrypted decoder layers
    with their refreshes (bootstraps included) on REFRESH_PARAMS (or
    ``params``, CtS/StC budget ``budget``, with the softmax normalisers' and
    the slim RMSNorm's refreshes as measure_fm_layers takes them), every key
    and every layer's weights resident on the device, the final hidden state
    decrypted and the final token's logits computed in the clear (exact final
    RMSNorm and LM head).  Weights N(0, 0.02) (embedding, projections, LM
    head) in a Hadamard-rotated residual basis, drawn on the GPU from seeded
    generators.  Each layer's series intervals are calibrated on a second
    random token sequence in plaintext.  Logits are compared with the fp64
    forward (exact RMSNorm, SiLU and softmax) and with the fp64 forward that
    uses the fitted series."""
    import torch

    from easyfhe import fhe
    from feature_major import FeatureMajorPrefillLayout
    from easyfhe.bs import openfhe as bs
    from feature_major.layer import (DecoderLayerWeights, decoder_layer_rotations,
                                     normaliser_program, refreshed_layer_depths,
                                     refreshed_layer_programs, rmsnorm_slim_program)
    from feature_major.model import (approximations_for, embed_tokens, final_logits,
                                     layer_ranges, prefill_fhe)

    params = REFRESH_PARAMS if params is None else params
    budget = tuple(int(v) for v in budget)
    # contexts dropped by earlier work in this process give their device
    # memory back before this one sizes its pool against what is free
    gc.collect()
    torch.cuda.empty_cache()
    free_at_start = torch.cuda.mem_get_info()[0]
    T, D, H, KV, hd, I = 128, 4096, 32, 8, 128, 14336
    lay = FeatureMajorPrefillLayout(seq_len=T, hidden_dim=D, slots=32768)
    spec = fhe.CKKSContextSpec(**params, seed=seed,
                               rotations=decoder_layer_rotations(lay, H, hd))
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    ctx.synchronize()
    setup_s = time.perf_counter() - t0

    t0 = time.perf_counter()
    dev = torch.device("cuda")
    R = torch.tensor(randomized_hadamard(D, seed + 1), dtype=torch.float64, device=dev)

    def draw(gen, *shape):
        return torch.randn(*shape, generator=gen, dtype=torch.float64, device=dev) * 0.02

    g0 = torch.Generator(device=dev).manual_seed(seed)
    embed = (draw(g0, vocab, D) @ R).cpu().numpy()
    lm_head = (draw(g0, vocab, D) @ R).cpu().numpy()
    rng = np.random.default_rng(seed)
    test_ids, cal_ids = rng.integers(0, vocab, T), rng.integers(0, vocab, T)
    x_test = embed_tokens(test_ids, embed)
    x_cal = torch.tensor(embed_tokens(cal_ids, embed), device=dev)
    x_ex = torch.tensor(x_test, device=dev)
    x_po = x_ex.clone()
    layers, bounds, ranges = [], [], []
    try:
        for li in range(int(n_layers)):
            g = torch.Generator(device=dev).manual_seed(seed * 1000 + 7 + li)
            w = dict(q=draw(g, D, D) @ R, k=draw(g, KV * hd, D) @ R, v=draw(g, KV * hd, D) @ R,
                     o=R.T @ draw(g, D, D), gate=draw(g, I, D) @ R, up=draw(g, I, D) @ R,
                     down=R.T @ draw(g, D, I))
            f = _TorchLayer(w, H=H, KV=KV, hd=hd, T=T)
            x_next, h1, gate, sc = f(x_cal)
            r = layer_ranges(x_cal.cpu().numpy(), h1.cpu().numpy(), gate.cpu().numpy(),
                             sc.cpu().numpy())
            ap, bound = approximations_for(r)
            x_cal = x_next
            x_ex = f(x_ex)[0]
            x_po = f(x_po, ap)[0]
            host = {k: v.cpu().numpy() for k, v in w.items()}
            del w, f, h1, gate, sc
            layers.append(DecoderLayerWeights(host["q"], host["k"], host["v"], host["o"],
                                              host["gate"], host["up"], host["down"], heads=H,
                                              kv_heads=KV, head_dim=hd, intermediate=I,
                                              approx=ap, layout=lay, context=ctx))
            bounds.append(bound)
            ranges.append(r)
            print(f"prepared layer {li}: residual bound {bound:.3g}, mean square "
                  f"{r.input_mean_square[0]:.3g}..{r.post_attention_mean_square[1]:.3g}, "
                  f"scores {r.score_min:.2f}..{r.score_max:.2f}", file=sys.stderr, flush=True)
        want_exact = x_ex.cpu().numpy()
        want_poly = x_po.cpu().numpy()
        del x_cal, x_ex, x_po, R
        torch.cuda.empty_cache()
        ctx.synchronize()
        prep_s = time.perf_counter() - t0
        # every layer's series have the same degrees, hence the same depths
        if len({refreshed_layer_depths(w_.approx, T, refresh_normalisers=refresh_normalisers,
                                       slim_rmsnorm=slim_rmsnorm) for w_ in layers}) != 1:
            raise ValueError("layers with different depths need programs of their own")
        t0 = time.perf_counter()
        ap0 = layers[0].approx
        prog, res_prog = refreshed_layer_programs(ctx, ap0, T, log_slots=15, level_budget=budget,
                                                  refresh_normalisers=refresh_normalisers,
                                                  slim_rmsnorm=slim_rmsnorm)
        lam_prog = (normaliser_program(ctx, ap0, T, log_slots=15, level_budget=budget)
                    if refresh_normalisers else None)
        rms_prog = (rmsnorm_slim_program(ctx, ap0, T, log_slots=15, level_budget=budget,
                                         refresh_normalisers=refresh_normalisers)
                    if slim_rmsnorm else None)
        ctx.synchronize()
        setup_s += time.perf_counter() - t0

        packed = lay.pack(x_test)
        # the lowest level a refresh takes on this chain
        start = bs.input_limbs(ctx)
        cts = [client.encrypt(packed[i], cur_limbs=start, enc_id=700000 + i)
               for i in range(lay.cipher_count)]
        ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
        ctx.synchronize()
        ctx.audit(reset=True)
        ev0.record()
        t0 = time.perf_counter()
        allocs, mems, free = [], [], []

        def on_layer(i, s):
            # the pool's device allocations so far: a layer that grows the
            # pool pays its hipMalloc calls; its live / cached bytes; and the
            # device memory nobody holds
            m = ctx.memory_info()
            allocs.append(int(m["device_allocations"]))
            mems.append([round(m["live_bytes"] / 2**30, 1), round(m["cached_bytes"] / 2**30, 1),
                         round(m["segment_bytes"] / 2**30, 1)])
            free.append(round(torch.cuda.mem_get_info()[0] / 2**30, 1))
            print(f"layer {i}: {s:.2f} s, {allocs[-1]} device allocations, live / cached / "
                  f"segments {mems[-1]} GiB, device free {free[-1]} GiB", file=sys.stderr,
                  flush=True)

        res = prefill_fhe(cts, layers, crypto_context=ctx, program=prog,
                          residual_program=res_prog, residual_bounds=bounds,
                          normaliser_program=lam_prog, rmsnorm_program=rms_prog,
                          on_layer=on_layer)
        ev1.record()
        ctx.synchronize()
        wall = time.perf_counter() - t0
        audit = ctx.audit(reset=True)
        for c in cts:
            c.release()
        got = lay.unpack(np.stack([client.decrypt(o) for o in res.ciphers]))
        out_limbs = int(res.ciphers[0].state.cur_limbs)
        res.release()
    finally:
        for w_ in layers:
            w_.close()
    mem = ctx.memory_info()
    L, alpha = ctx.L, ctx.alpha
    log_qp = sum(int(q).bit_length() for q in ctx.primes())
    ctx.close()
    ones = np.ones(D)
    lg = final_logits(got, norm_weight=ones, lm_head=lm_head)
    lg_exact = final_logits(want_exact, norm_weight=ones, lm_head=lm_head)
    lg_poly = final_logits(want_poly, norm_weight=ones, lm_head=lm_head)
    top5 = lambda v: set(np.argsort(v)[-5:].tolist())  # noqa: E731
    return {
        "seconds": round(wall, 2),
        "seconds_per_layer": round(wall / max(1, int(n_layers)), 3),
        "gpu_event_seconds": round(ev0.elapsed_time(ev1) / 1000.0, 2),
        "layers": int(n_layers),
        "layer_s": [round(v, 2) for v in res.layer_seconds],
        "device_allocations_after_layer": allocs,
        "live_cached_segment_gib_after_layer": mems,
        "device_free_gib_after_layer": free,
        "device_free_gib_at_start": round(free_at_start / 2**30, 1),
        "roofline": audit_roofline(audit, wall, int(n_layers), "layer"),
        "workload": f"{n_layers}-layer Llama-3-8B prefill (d=4096, 32/8 heads x 128, SwiGLU "
                    f"14336, vocab {vocab}) over 128 random tokens in 16 ciphertexts of 8 lanes, "
                    "every layer boundary encrypted, bootstraps included (24 per layer"
                    + (", plus 3 softmax normaliser refreshes" if refresh_normalisers else "")
                    + (", plus 1 slim RMSNorm refresh" if slim_rmsnorm else "")
                    + f"), N=2^16, Q=1x{params['first_mod']}b+{L - 1}x{params['dcrt_bits']}b, "
                    f"dnum={params['dnum']}, P={alpha}x{params['special_bits']}b, CtS/StC budget "
                    f"{budget}; final token's logits in the clear",
        "log_qp_bits": log_qp,
        # N / log QP scaled from the standard's 128-bit point (log QP <= 1747
        # at N = 2^16, uniform ternary): an upper estimate for h = 192 secrets
        "security_estimate_bits": round(128 * 1747 / log_qp),
        "logits_max_abs_err_vs_fp64_exact": float(np.abs(lg - lg_exact).max()),
        "logits_max_abs_err_vs_fp64_series": float(np.abs(lg - lg_poly).max()),
        "logits_abs_max": float(np.abs(lg_exact).max()),
        "top1_match_exact": bool(int(np.argmax(lg)) == int(np.argmax(lg_exact))),
        "top5_overlap_exact": len(top5(lg) & top5(lg_exact)),
        "hidden_max_abs_err_vs_fp64_series": float(np.abs(got - want_poly).max()),
        "hidden_max_abs_err_vs_fp64_exact": float(np.abs(got - want_exact).max()),
        "hidden_abs_max": float(np.abs(want_exact).max()),
        "output_limbs": out_limbs,
        "setup_s": round(setup_s, 2),
        "weights_and_calibration_s": round(prep_s, 2),
        "residual_bounds": [round(b, 2) for b in bounds],
        "score_max": round(max(r.score_max for r in ranges), 2),
        "device_memory": _memory_summary(mem),
    }


def keyswitch_step(ctx, cts, levels: int) -> list:
    """One step of the key-switch workload: rotations by 2^0 .. 2^14 of every
    ciphertext (chained), then `levels` levels of HMult + relinearise +
    rescale; intermediates are released as they are consumed."""
    from easyfhe import fhe

    cur = cts
    for r in ROTATIONS:
        nxt = fhe.homo_rotate_many(cur, r, ctx)
        if cur is not cts:
            for c in cur:
                c.release()
        cur = nxt
    for _ in range(levels):
        nxt = fhe.homo_mul_relin_rescale_many(cur, cur, ctx)
        for c in cur:
            if c not in cts:
                c.release()
        cur = nxt
    return cur


def ks_profile(spec, n_cts: int, levels: int) -> int:
    """Exactly one key-switch step over n_cts ciphertexts (after set-up), then
    three device copies of one 36 MiB ciphertext (the counters' calibration
    kernel): the program rocprofv3 counter runs of the step use."""
    from easyfhe import fhe

    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    cts = [client.encrypt(rng.uniform(-1, 1, slots), slots=slots, enc_id=i + 1)
           for i in range(n_cts)]
    ctx.synchronize()
    for c in keyswitch_step(ctx, cts, min(levels, ctx.L - 2)):
        c.release()
    copies = [cts[0].deep_copy() for _ in range(3)]
    ctx.synchronize()
    print(json.dumps({"keyswitch_steps": 1, "ciphertexts": n_cts,
                      "copy_bytes": 2 * ctx.L * ctx.N * 8, "copies": len(copies)}), flush=True)
    return 0


def int_peaks(ctx) -> dict:
    """Device-wide rates of the register-only probes (ops/s): the fp64-path
    modular product (limbs below 2^45), the 64-bit Shoup product, fp64 FMA."""
    import ctypes

    from easyfhe import _native

    out = {}
    for kind, name in ((0, "fp64_modmul"), (1, "shoup64_modmul"), (2, "fp64_fma")):
        v = ctypes.c_double()
        _native.check(_native.lib.ckks_int_peak(ctx.handle, kind, ctypes.byref(v)))
        out[name] = v.value
    return out


# kernel groups whose modular operations run on the fp64 path (40-bit limbs)
_INT_GROUPS = ("basis_convert", "basis_convert_rescale", "key_inner", "key_inner_multi",
               "mac", "mac_many", "mac_table", "tensor", "lincomb")


def kernel_table(prof: dict, peaks: dict) -> dict:
    """Per kernel group of one profiled step: launches, device ms, share of the
    summed kernel time, algorithmic bytes / time against the 8 TB/s peak and,
    for the modular-arithmetic groups, operations / time against the fp64-path
    probe."""
    total = sum(v["ms"] for v in prof.values()) or 1.0
    out = {}
    for name, v in sorted(prof.items(), key=lambda kv: -kv[1]["ms"]):
        t = max(v["ms"], 1e-9) * 1e-3
        row = {"launches": v["launches"], "ms": round(v["ms"], 3),
               "share": round(v["ms"] / total, 4),
               "gbs": round(v["bytes"] / t / 1e9, 1),
               "hbm_frac": round(v["bytes"] / t / 1e9 / HBM_PEAK_GBS, 4)}
        if name in _INT_GROUPS:
            rate = v["ops"] / t
            row["gmodops"] = round(rate / 1e9, 1)
            row["int_frac"] = round(rate / peaks["fp64_modmul"], 4)
        out[name] = row
    return out


def measure_matvec_config(iters: int = 20) -> dict:
    """The CPU matvec workload on the device: N = 2^13, 4096 slots, 4 x 40-bit
    limbs + one 60-bit special prime, scale 2^40, 128 x 128 W and x
    uniform[-1, 1] from seed 0, BSGS B = 16, G = 8, 32 token lanes; one
    matvec = hoisted babies + MAC + giant Horner + rescale, averaged over
    `iters` after a warm-up; decrypted against fp64 W x."""
    from easyfhe import fhe

    D, lanes, B, G = 128, 32, 16, 8
    rots = tuple(lanes * b for b in range(1, B)) + (B * lanes,)
    spec = fhe.CKKSContextSpec(depth=3, log_n=13, dnum=4, dcrt_bits=40, first_mod=40,
                               special_bits=60, seed=0, rotations=rots)
    t0 = time.perf_counter()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    W = rng.uniform(-1, 1, (D, D))
    x = rng.uniform(-1, 1, D)
    packed = np.zeros(slots)
    packed[np.arange(D) * lanes] = x
    feat = np.arange(slots) // lanes
    rows = np.stack([W[(feat - g * B) % D, (feat + b) % D] for g in range(G) for b in range(B)])
    pts = fhe.encode_rows(ctx, rows, limbs=ctx.L, scale=ctx.scale_at(ctx.L), slots=slots)
    ct = client.encrypt(packed, slots=slots, enc_id=41)
    ctx.synchronize()
    setup = time.perf_counter() - t0
    offsets = [lanes * b for b in range(B)]

    def one():
        acc = fhe.hoisted_mac_sum(ct, offsets, pts, B * lanes, G, ctx)
        out = fhe.rescale(acc, ctx)
        acc.release()
        return out

    one().release()
    ctx.synchronize()
    ev0, ev1 = fhe_event(ctx), fhe_event(ctx)
    ev0.record()
    t0 = time.perf_counter()
    for _ in range(iters - 1):
        one().release()
    out = one()
    ev1.record()
    ctx.synchronize()
    wall = (time.perf_counter() - t0) / iters
    err = float(np.abs(client.decrypt(out)[np.arange(D) * lanes] - W @ x).max())
    res = {"workload": "BSGS matvec, N=2^13, 4x40b limbs + 1x60b special, 128x128 W, B=16, G=8, "
                       "seed 0", "ms_per_matvec": round(wall * 1e3, 3),
           "gpu_event_ms_per_matvec": round(ev0.elapsed_time(ev1) / iters, 3),
           "setup_s": round(setup, 3), "max_abs_err_vs_fp64": err}
    ctx.close()
    return res


def bootstrap_bench(spec, args) -> int:
    """The bootstrap workload alone, as its own JSON line."""
    from easyfhe import fhe

    spec.rotations = ()
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    b = measure_bootstrap(client, ctx, args.boot_cts, args.boot_group, args.budget, args.warmup)
    sparse = measure_bootstrap(client, ctx, args.boot_cts, args.boot_group, args.budget,
                               args.warmup, log_slots=7)
    result = {
        "metric": "bootstrap/s @N=2^16",
        "value": b["value"],
        "unit": "bootstrap/s",
        "n_gpus": 1,
        "steps": b["ciphertexts"],
        "warmup": max(1, args.warmup),
        "ms_per_step": b["ms_per_bootstrap"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64",
        "data": "synthetic",
        "config": {
            "workload": f"full-slot bootstrap, N=2^16, Q=1x60b+35x40b, dnum=3, P=12x44b; "
                        f"{b['ciphertexts']} ciphertexts at one limb; CtS/StC budget "
                        f"{tuple(b['budget'])}",
        },
        "bootstrap": b,
        "bootstrap_sparse_128": sparse,
    }
    print(json.dumps(result), flush=True)
    return 0


def ntt_profile(spec, n_cts: int) -> int:
    """Three forward+inverse batch NTTs over n_cts ciphertexts at 36 limbs,
    then three device copies of one 36 MiB ciphertext."""
    from easyfhe import _native, fhe

    spec.rotations = ()
    spec.relin_key = False
    client, ctx = fhe.generate_client_context(spec, device="cuda:0")
    slots = ctx.max_slots
    rng = np.random.default_rng(0)
    cts = [client.encrypt(rng.uniform(-1, 1, slots), slots=slots, enc_id=i + 1)
           for i in range(n_cts)]
    batch = fhe_ptrs(cts)
    for _ in range(3):
        _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 0))
        _native.check(_native.lib.ckks_ntt_many(ctx.handle, batch, len(cts), 1))
    copies = [cts[0].deep_copy() for _ in range(3)]
    ctx.synchronize()
    print(json.dumps({"ntt_limb_polys_per_call": len(cts) * 2 * ctx.L,
                      "copy_bytes": 2 * ctx.L * ctx.N * 8, "copies": len(copies)}), flush=True)
    return 0


def fhe_event(ctx):
    from easyfhe.cuda import Event

    return Event(enable_timing=True, context=ctx)


def fhe_ptrs(cts):
    from easyfhe._native import ptr_array

    return ptr_array([c.handle for c in cts])


if __name__ == "__main__":
    sys.exit(main())
