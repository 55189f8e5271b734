#!/usr/bin/env python3
"""Benchmark: online secure samples/s of the two-party affinity forward on one
MI355X (bw=32, scale 12, B=64 molecules x 140 atoms, all FSS keys resident in
HBM), plus the DCF-evaluation kernel's roofline and the CPU oracle baseline.

One step = one online forward of both parties over one batch of B synthetic
molecules (inputs and keys resident in HBM; keygen is the offline dealer and
is not timed).  Prints one JSON line.
"""
import argparse
import hashlib
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "idash26-track3_amd"))

METRIC = "online secure samples/s (bw=32, B=64, 1 GPU); DCF evals/s; % roofline"


def affinity_metric(bw, B):
    """The headline metric's name for a ring width and batch (METRIC itself at bw=32, B=64)."""
    return f"online secure samples/s (bw={bw}, B={B}, 1 GPU); DCF evals/s; % roofline"

# Peak integer VALU rate of MI355X: 256 CUs x 4 SIMD x 16 lanes x 2.4 GHz.
VALU_PEAK_TOPS = 256 * 64 * 2.4e9 / 1e12
# Peak LDS read rate: 128 bytes per clock per CU (a 64-lane ds_read_b32 in two
# clocks), 256 CUs x 2.4 GHz.
LDS_PEAK_TBS = 256 * 128 * 2.4e9 / 1e12
HBM_PEAK_GBS = 8000.0
# Ring multiply-adds per second at the peak of each GEMM path: the int8 matrix
# cores (5.0 POP/s dense = 2.5 P int8 MAC/s) spend 16 int8 MACs per Z_2^32 MAC
# (four digit bytes x four shift MFMAs) and 64 per Z_2^64 MAC (eight x eight);
# the VALU path 2 instructions per MAC.
GEMM_PEAK_TMACS = {"mfma32": 5.0e3 / 2 / 16, "mfma64": 5.0e3 / 2 / 64, "valu": VALU_PEAK_TOPS / 2}
# VALU instructions per AES call of the DCF walk (one tree level: the unrolled
# cipher, sigma, feed-forward and the level update), counted in the gfx950 ISA
# of this build: hipcc --cuda-device-only -S csrc/gates.hip, level-loop block
# of k_tr_eval<uint32_t, NT, REP> for each LDS table variant.
# HBM bytes per k_tr_eval launch, measured with rocprofv3 --pmc FETCH_SIZE and
# WRITE_SIZE (one run each) on this bench command, mean over the launches of the
# forward, each counter scaled by its reading on a plain 1 GiB copy
# (bench.py --workload copy: FETCH_SIZE x 2.0, WRITE_SIZE x 1.0).  A measurement
# holds only for the kernel sources and the model's launch sequence it was taken
# on: it is keyed by the digest of those sources (kernel_digest(): the gate
# kernels and csrc/model.hip, which decides the launches) and the workload, and the line reports null
# when the current sources or workload have no measurement.  Each entry names
# the profile summary under profiles/ that it comes from.
TRAFFIC_MEASURED = {
    ("a82189763dae", "perm32x2_b512", 64, 32, 3, 0): {
        "bytes_per_launch": 70798343, "profile": "profiles/k_tr_eval_affinity_bw32_B64.md"},
}
KERNEL_SOURCES = ("csrc/gates.hip", "csrc/launch_util.h", "csrc/kernels.h", "csrc/dcf_dev.h", "csrc/aes_dev.h",
                  "csrc/mpcx_core.h", "csrc/model.hip")
SLACK_DESC = {1: ", GCN products H.W^T truncated with the slack gate",
              2: ", GCN products and aggregations truncated with the slack gate",
              3: ", every layer truncation local (LocalARS, the reference's default truncation; not bit-exact)"}
VALU_OPS_PER_AES = {"perm32x2_b512": 318, "perm64_b512": 390, "perm64_b1024": 390, "t4_rep32_b1024": 452}
# The both-party form (one thread per element runs both parties' walks) issues
# 617 VALU instructions per level loop of two AES calls on the T0/T1 table: a
# forward that mixes the two forms converts its AES calls at the lower count,
# so its VALU rate is a lower bound.
VALU_OPS_PER_AES_MIXED = dict(VALU_OPS_PER_AES, perm32x2_b512=308.5)
# LDS table bytes read per AES call: 16 four-byte lookups per round, ten rounds
# (the same level-loop blocks: 160 ds_read_b32 in every variant)
LDS_BYTES_PER_AES = 160 * 4


def lds_colimit(aes_per_s):
    """The T-table reads of the same AES work against the LDS peak: the second
    limit of the DCF kernel (its level loop issues about two VALU instructions
    per table read, and a read takes two LDS clocks)."""
    tbs = aes_per_s * LDS_BYTES_PER_AES / 1e12
    return {"resource": "lds", "achieved": round(tbs, 2), "peak": round(LDS_PEAK_TBS, 2), "unit": "TB/s",
            "frac": round(tbs / LDS_PEAK_TBS, 4)}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def kernel_digest():
    """First 12 hex digits of the SHA-256 of the DCF kernel's sources."""
    h = hashlib.sha256()
    for rel in KERNEL_SOURCES:
        with open(os.path.join(ROOT, "idash26-track3_amd", rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:12]


def host_cpu():
    """The host CPU the baseline runs on: model name and logical CPUs visible."""
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count()
    return {"cpu_model": model, "nproc": avail, "cpu_count": os.cpu_count()}


def cpu_fields(orc):
    """cores and host description of a CPU-baseline object."""
    d = {"cores": orc.get_threads()}
    d.update(host_cpu())
    return d


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--bw", type=int, default=32)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--cpu-samples", type=int, default=8, help="molecules per CPU baseline evaluation")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="minimum timed CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--aes-variant", type=int, default=-1)
    ap.add_argument("--aes-block", type=int, default=0,
                    help="threads per DCF workgroup (0: the variant's own; a multiple of 128 up to 1024)")
    ap.add_argument("--both-aes", type=int, default=-1,
                    help="mpcx_set_both_party_aes: longest gate (AES calls per element and party) in the "
                         "both-party form (-1: the library's default)")
    ap.add_argument("--lanes", type=int, default=3, help="concurrent sub-batches, each on its own stream")
    ap.add_argument("--slack", type=int, default=0, choices=(0, 1, 2, 3),
                    help="slack truncations of the GCN (exact while the values lie in half the signed ring): "
                         "0 none (exact truncation over the whole ring), 1 the products H.W^T, 2 also the "
                         "aggregation A.XW + bias (then a small-domain ReLU); 3 every layer truncation local "
                         "(LocalARS, the reference's default; not bit-exact, bw=64 only in practice)")
    ap.add_argument("--xw-slack", action="store_true", help="same as --slack 1")
    ap.add_argument("--workload", choices=("affinity", "relu", "adjnorm", "copy", "shim"), default="affinity",
                    help="affinity: the secure forward (default); relu: secure ReLU over --n elements (bw=32); "
                         "adjnorm: secure adjacency normalisation of B=1024 graphs (bw=32); copy: a 1 GiB "
                         "elementwise kernel (b = a + 1 over 2^28 int32), the HBM reference for the PMC byte "
                         "counters and the achievable copy bandwidth")
    ap.add_argument("--n", type=int, default=1 << 24, help="elements of the relu workload")
    ap.add_argument("--stream", action="store_true",
                    help="bw=64 streamed-key workload: micro-batches of --batch (default 256) over --total samples, "
                         "keys in pinned host memory copied through two device slots")
    ap.add_argument("--total", type=int, default=8192, help="samples of the streamed workload")
    ap.add_argument("--slot-gb", type=float, default=16.0, help="device slot size per party (streamed workload)")
    ap.add_argument("--distinct", type=int, default=4, help="distinct input micro-batches cycled (streamed workload)")
    ap.add_argument("--key-files", default=None,
                    help="streamed workload from key files in this directory: --sets distinct dealer key sets are "
                         "appended to two files and every micro-batch reads the next set (cycling)")
    ap.add_argument("--sets", type=int, default=4, help="key sets in the key files")
    ap.add_argument("--party", action="store_true",
                    help="party mode: the two parties as two processes on the one GPU, exchanging over a Unix "
                         "socket (the reference's deployment); one lane per party")
    ap.add_argument("--party-child", type=int, default=-1, help=argparse.SUPPRESS)
    ap.add_argument("--party-sock", default="", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.xw_slack:
        args.slack = max(args.slack, 1)

    if args.gpus != 1:
        print(f"bench.py measures one GPU only (every box here has one GPU); got --gpus {args.gpus}.",
              file=sys.stderr)
        sys.exit(2)

    if args.party_child >= 0:
        return run_party_child(args)
    if args.party:
        return run_party(args)
    if args.stream:
        return run_stream(args)
    if args.workload == "relu":
        return run_relu(args)
    if args.workload == "adjnorm":
        return run_adjnorm(args)
    if args.workload == "copy":
        return run_copy(args)
    if args.workload == "shim":
        return run_shim(args)

    import numpy as np

    import mpcx
    import synth

    B = args.batch
    dims = synth.Dims(bw=args.bw, slack=args.slack)
    t0 = time.time()
    wl = synth.workload(B, dims, seed=args.seed)
    log(f"[bench] workload B={B} bw={args.bw} generated in {time.time() - t0:.1f}s")

    ctx = mpcx.Ctx(bw=args.bw, scale=dims.s)
    if args.aes_variant >= 0:
        ctx.set_aes_variant(args.aes_variant, args.aes_block)
    if args.both_aes >= 0:
        ctx.set_both_party_aes(args.both_aes)
    model = mpcx.Model(ctx, dims, wl.W, lanes=args.lanes)
    key_bytes = model.key_bytes(B)
    t0 = time.time()
    model.keygen(B, 0xC0FFEE + args.seed)
    log(f"[bench] GPU dealer: {2 * key_bytes / 1e9:.2f} GB of keys (both parties) in {time.time() - t0:.1f}s")
    model.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)

    for _ in range(args.warmup):
        model.forward(B)
    ctx.sync()
    log(f"[bench] warmup {args.warmup} done")
    ctx.reset_counters()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        model.forward(B)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    out = model.output(B)
    bytes_per_fwd = ctx.bytes_exchanged / max(args.steps, 1)
    rounds_per_fwd = ctx.rounds / max(args.steps, 1)
    ms_per_step = 1e3 * elapsed / args.steps
    value = B * args.steps / elapsed
    log(f"[bench] {args.steps} steps in {elapsed:.3f}s -> {ms_per_step:.2f} ms/step, {value:.1f} samples/s")

    # one profiled forward: HIP events around every DCF-evaluation launch, the
    # lanes run one after another so that each launch is timed alone
    model.profile(True)
    model.forward(B)
    prof = model.profile_read()
    model.profile(False)
    dcf_ms = prof["ms"]
    variant = ctx.aes_variant_name()
    # rates over the timed step (the work of one forward, whatever overlaps it)
    step_s = ms_per_step / 1e3
    dcf_evals_per_s = prof["elements"] / step_s
    aes_per_s = prof["aes_calls"] / step_s
    key_gbs = prof["hbm_bytes"] / step_s / 1e9
    valu_per_aes = (VALU_OPS_PER_AES_MIXED if args.bw == 32 else VALU_OPS_PER_AES).get(variant, float("nan"))
    step_tops = aes_per_s * valu_per_aes / 1e12
    # rate of the launches alone (profiled forward, lanes one after another)
    launch_aes_per_s = prof["aes_calls"] / (dcf_ms / 1e3) if dcf_ms > 0 else 0.0
    achieved_tops = launch_aes_per_s * valu_per_aes / 1e12
    gemm_path = "valu" if os.environ.get("MPCX_GEMM") == "valu" else f"mfma{args.bw}"
    gemm_tmacs = prof["gemm_macs"] / (prof["gemm_ms"] / 1e3) / 1e12 if prof["gemm_ms"] > 0 else 0.0
    digest = kernel_digest()
    tm = TRAFFIC_MEASURED.get((digest, variant, B, args.bw, args.lanes, args.slack))
    traffic = tm["bytes_per_launch"] if tm else None
    traffic_src = tm["profile"] if tm else f"no PMC measurement for kernel sources {digest} and this workload"
    log(f"[bench] DCF gate launches: {prof['launches']} per forward ({dcf_ms:.2f} ms alone); over the step "
        f"{dcf_evals_per_s / 1e9:.3f} G evals/s, {aes_per_s / 1e9:.2f} G AES/s")

    result = {
        "metric": affinity_metric(args.bw, B),
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32" if args.bw == 32 else "u64",
        "data": "synthetic molecules (random trees + ring closures, 10-60 atoms), Kaiming-normal weights",
        "config": {"workload": f"two-party secure affinity forward, bw={args.bw} s=12, B={B} molecules x "
                               f"{dims.n_nodes} atoms, GCN 78-78-156-312, FC 312-1024-128, fusion 256-1024-512-1, "
                               f"FSS keys resident in HBM, {args.lanes} concurrent sub-batches"
                               + SLACK_DESC.get(args.slack, ""),
                   "B": B, "n_nodes": dims.n_nodes, "bw": args.bw, "scale": dims.s, "lanes": args.lanes,
                   "slack": args.slack},
        "dcf_evals_per_s": round(dcf_evals_per_s, 1),
        "aes_blocks_per_s": round(aes_per_s, 1),
        "bytes_exchanged_per_sample": round(bytes_per_fwd / B, 1),
        "rounds_per_step": rounds_per_fwd,
        "key_bytes_per_sample_per_party": round(key_bytes / B, 1),
        # The DCF gate kernel's VALU work of every launch of a timed step over
        # the timed step itself: the lanes' launches overlap each other and the
        # GEMM and exchange kernels, so this is the kernel's rate as the timed
        # configuration runs it (a lower bound on its rate while it runs).
        "roofline": {
            "kernel": f"k_tr_eval (DCF gate evaluation of both parties, AES-128 T-tables in LDS, {variant}): "
                      f"VALU work of all {prof['launches']} launches of a step over the timed step",
            "bound": "valu",
            "achieved": round(step_tops, 3),
            "peak": round(VALU_PEAK_TOPS, 2),
            "unit": "TOP/s",
            "frac": round(step_tops / VALU_PEAK_TOPS, 4),
            "traffic": traffic,
            "traffic_unit": "HBM bytes per launch (FETCH_SIZE + WRITE_SIZE, mean over a forward's launches)",
            "traffic_source": traffic_src,
            "algorithmic_bytes_per_launch": round(prof["hbm_bytes"] / max(prof["launches"], 1)),
            "launches_per_step": prof["launches"],
            "aes_calls_per_step": prof["aes_calls"],
            "valu_ops_per_aes": valu_per_aes,
            "co_limit": lds_colimit(aes_per_s),
            "kernel_digest": digest,
        },
        # The same launches timed one by one (HIP events on the launch streams)
        # in a profiled forward whose lanes run one after another: the kernel's
        # rate alone, per launch.  rocprofv3 --kernel-trace lists these launches
        # under their own instantiation k_tr_eval<..., 1>.
        "roofline_launch": {
            "kernel": "k_tr_eval, profiled forward (lanes one after another, every launch timed alone)",
            "launches": prof["launches"],
            "avg_launch_us": round(1e3 * dcf_ms / max(prof["launches"], 1), 2),
            "ms_per_forward": round(dcf_ms, 3),
            "bound": "valu",
            "achieved": round(achieved_tops, 3),
            "peak": round(VALU_PEAK_TOPS, 2),
            "unit": "TOP/s",
            "frac": round(achieved_tops / VALU_PEAK_TOPS, 4),
            "co_limit": lds_colimit(launch_aes_per_s),
        },
        "roofline_gemm": {
            "kernel": f"ring GEMMs ({gemm_path}: public-weight products and SxS Beaver products, "
                      f"{prof['gemm_sections']} sections of the profiled forward"
                      + ("; products of at most 4 columns on the VALU dot kernel)" if gemm_path != "valu" else ")"),
            "bound": "valu" if gemm_path == "valu" else "mfma",
            "achieved": round(gemm_tmacs, 3),
            "peak": round(GEMM_PEAK_TMACS[gemm_path], 2),
            "unit": "T ring MAC/s",
            "frac": round(gemm_tmacs / GEMM_PEAK_TMACS[gemm_path], 4),
            "ms_per_step": round(prof["gemm_ms"], 3),
            "ring_macs_per_step": prof["gemm_macs"],
        },
        "roofline_hbm": {
            "kernel": "k_tr_eval key stream (algorithmic bytes of a forward over the timed step)",
            "bound": "hbm",
            "achieved": round(key_gbs, 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(key_gbs / HBM_PEAK_GBS, 4),
        },
    }

    # ---- oracle: bit-exact check of all B outputs and the timed CPU baseline ----
    try:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import orc
        d = dims
        od = orc.make_dims(bw=d.bw, s=d.s, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                           fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale,
                           slack=d.slack)
        want, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, wl.W)
        result["bit_exact"] = bool(code == 0 and np.array_equal(want, out))
        if code == 0:  # outputs in units of 2^-s (0 unless the truncation is local)
            result["max_abs_err_lsb"] = int(np.max(np.abs(out.astype(np.int64) - want)))
        if not args.no_cpu:
            nb = min(args.cpu_samples, B)
            sl = synth.workload(nb, dims, seed=args.seed)  # same generator, first nb molecules
            k0, k1 = orc.model_keygen(od, nb, 99, sl.W)
            sh = sl.shares
            cwant, _ = orc.plain_forward(od, sl.X, sl.A, sl.mask, sl.prot, sl.W)
            reps, ct, exact, cerr = 0, 0.0, True, 0
            while ct < args.cpu_seconds or reps == 0:
                t0 = time.perf_counter()
                cout, _ = orc.model_eval(od, nb, sl.W, k0, k1, *sh["x"], *sh["a"], *sh["m"], sl.prot)
                ct += time.perf_counter() - t0
                reps += 1
                exact = exact and bool(np.array_equal(cout, cwant))
                cerr = max(cerr, int(np.max(np.abs(cout - cwant))))
            result["cpu_baseline"] = {
                "value": round(nb * reps / ct, 3),
                "unit": "samples/s",
                **cpu_fields(orc),
                "kind": "port",
                "sample": f"{reps} x {nb} molecules of the same workload: two-party online eval (both parties, "
                          f"same gates and key format) in oracle/ C with AES-NI + OpenMP, {ct:.1f}s",
                "bit_exact": exact,
                "max_abs_err_lsb": cerr,
            }
            log(f"[bench] CPU oracle: {reps}x{nb} samples in {ct:.2f}s on {orc.get_threads()} threads")
    except Exception as e:  # the product number stands without the checker
        log(f"[bench] oracle unavailable: {e}")
        result.setdefault("bit_exact", None)

    print(json.dumps(result), flush=True)
    model.close()
    ctx.close()


def run_stream(args):
    """Streamed key arena: bw=64 (scale 12), micro-batches of B molecules over
    `total` samples.  The dealer's keys for one micro-batch (both parties) sit in
    pinned host memory -- the keys of all `total` samples would not fit host RAM,
    so every micro-batch re-streams that key set with its own fresh inputs --
    and each forward copies them chunk by chunk into two device slots on a copy
    stream while the previous chunk computes.  Timed: input upload, forward and
    output download of every micro-batch."""
    import numpy as np

    import mpcx
    import synth

    B = args.batch if args.batch != 64 else 256
    bw = 64 if args.bw == 32 else args.bw
    dims = synth.Dims(bw=bw, slack=args.slack)
    nmb = max(1, args.total // B)
    wls = [synth.workload(B, dims, seed=args.seed + 100 * k) for k in range(args.distinct)]
    W = wls[0].W
    ctx = mpcx.Ctx(bw=bw, scale=dims.s)
    model = mpcx.Model(ctx, dims, W)
    kb = model.key_bytes(B)
    ku0, ku = model.unique_key_bytes(B, 0), model.unique_key_bytes(B, 1)
    h0 = h1 = None
    if args.key_files:
        # distinct dealer key sets in two files (party 0's arenas, party 1's
        # packed unique planes); each micro-batch reads the next set from disk
        os.makedirs(args.key_files, exist_ok=True)
        f0, f1 = os.path.join(args.key_files, "keys_p0.bin"), os.path.join(args.key_files, "keys_p1.bin")
        t0 = time.time()
        for k in range(args.sets):
            model.keygen(B, 0xBEEF + args.seed + k)
            model.write_keys(0, f0, packed=True, append=k > 0)
            model.write_keys(1, f1, packed=True, append=k > 0)
            log(f"[stream] key set {k + 1}/{args.sets} written ({(ku0 + ku) / 1e9:.1f} GB), {time.time() - t0:.1f}s")
        model.release_arena()
        model.attach_key_files(B, f0, f1, int(args.slot_gb * 2 ** 30))
        host_key_bytes = ku0 + ku
    else:
        t0 = time.time()
        model.keygen(B, 0xBEEF + args.seed)
        log(f"[stream] dealer: {2 * kb / 1e9:.1f} GB of keys for B={B} in {time.time() - t0:.1f}s")
        # both parties' packed keys: the correction words both parties hold are
        # stored once (party 0's), and the planes the dealer drew from a party's
        # own PRF key are expanded on the device after each chunk's copy
        t0 = time.time()
        h0, h1 = mpcx.PinnedBuffer(ku0), mpcx.PinnedBuffer(ku)
        log(f"[stream] pinned host buffers ({(h0.nbytes + h1.nbytes) / 1e9:.1f} GB) in {time.time() - t0:.1f}s")
        t0 = time.time()
        model.export_unique_keys(0, B, into=h0)
        model.export_unique_keys(1, B, into=h1)
        model.release_arena()
        log(f"[stream] keys exported to host in {time.time() - t0:.1f}s")
        model.attach_host_keys(B, h0, h1, int(args.slot_gb * 2 ** 30))
        host_key_bytes = h0.nbytes + h1.nbytes

    want = []
    try:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import orc
        d = dims
        od = orc.make_dims(bw=d.bw, s=d.s, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                           fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale,
                           slack=d.slack)
        for wl in wls:
            y, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, W)
            want.append(y if code == 0 else None)
    except Exception as e:  # the product number stands without the checker
        log(f"[stream] oracle unavailable: {e}")

    def step(k):
        wl = wls[k % len(wls)]
        model.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
        model.forward(B)
        return model.output(B)

    step(0)  # warmup
    exact = True
    ctx.reset_counters()
    h2d = 0
    t0 = time.perf_counter()
    outs = []
    for k in range(nmb):
        outs.append(step(k))
        h2d += model.stream_stats()["bytes_h2d"]
        if k % 8 == 7:
            log(f"[stream] {k + 1}/{nmb} micro-batches, {time.perf_counter() - t0:.1f}s")
    elapsed = time.perf_counter() - t0
    err = 0
    for k, out in enumerate(outs):
        w = want[k % len(want)] if want else None
        exact = exact and (w is not None and bool(np.array_equal(out, w)))
        if w is not None:
            err = max(err, int(np.max(np.abs(out.astype(np.int64) - w))))
    value = nmb * B / elapsed
    result = {
        "metric": f"online secure samples/s (bw={bw}, B={B} micro-batches, keys streamed from "
                  + ("key files" if args.key_files else "pinned host memory") + ", 1 GPU)",
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": nmb,
        "warmup": 1,
        "ms_per_step": round(1e3 * elapsed / nmb, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u64" if bw == 64 else "u32",
        "data": ("synthetic molecules; " + (f"{args.sets} dealer key sets in key files read in turn by the micro-batches"
                                            if args.key_files else
                                            "one dealer key set (pinned host memory) re-streamed for every micro-batch")
                 + ", fresh inputs per micro-batch"),
        "config": {"workload": f"two-party secure affinity forward, bw={bw} s=12, {nmb} micro-batches of B={B} "
                               f"molecules x {dims.n_nodes} atoms, keys streamed "
                               + ("from key files through pinned staging buffers and " if args.key_files else "")
                               + f"through two {args.slot_gb:g} GiB device slots per party"
                               + SLACK_DESC.get(args.slack, ""),
                   "B": B, "total": nmb * B, "bw": bw, "key_source": "files" if args.key_files else "pinned",
                   "slack": args.slack},
        "key_bytes_per_sample_per_party": round(kb / B, 1),
        "host_key_bytes_per_step": host_key_bytes,
        "key_h2d_bytes_per_step": h2d // nmb,
        "key_h2d_GBps": round(h2d / elapsed / 1e9, 2),
        "bytes_exchanged_per_sample": round(ctx.bytes_exchanged / (nmb * B), 1),
        "bit_exact": exact,
        "max_abs_err_lsb": err if want else None,
    }
    print(json.dumps(result), flush=True)
    model.close()
    ctx.close()
    for h in (h0, h1):
        if h is not None:
            h.free()


def run_party_child(args):
    """One party of the party-mode bench (a child of run_party): the dealer's
    keys (the GPU dealer run here, this party's key kept), the channel, W
    untimed forwards, a one-element exchange as a barrier, then K timed
    forwards; prints one JSON line."""
    import numpy as np

    import mpcx
    import synth

    party, B = args.party_child, args.batch
    dims = synth.Dims(bw=args.bw, slack=args.slack)
    wl = synth.workload(B, dims, seed=args.seed)
    ctx = mpcx.Ctx(bw=args.bw, scale=dims.s)
    dealer = mpcx.Model(ctx, dims, wl.W)
    dealer.keygen(B, 0xC0FFEE + args.seed)
    key = dealer.export_keys(party, B)
    prof = None
    if party == 0:  # the gates' work per forward, from one profiled one-process forward on the same keys
        dealer.set_inputs(B, *wl.shares["x"], *wl.shares["a"], *wl.shares["m"], wl.prot)
        dealer.profile(True)
        dealer.forward(B)
        prof = dealer.profile_read()
        dealer.profile(False)
    dealer.close()
    peer = mpcx.Peer.connect(party, args.party_sock, timeout_ms=120000)
    m = mpcx.Model(ctx, dims, wl.W)
    m.set_party(peer)
    m.import_party_key(B, key)
    sh = wl.shares
    m.set_party_inputs(B, sh["x"][party], sh["a"][party], sh["m"][party], wl.prot if party == 1 else None)
    for _ in range(args.warmup):
        m.forward(B)
    ctx.sync()
    bar = np.zeros(1, ctx.T)
    ctx.party_reconstruct(peer, bar)  # both parties leave this exchange together
    ctx.reset_counters()
    b0 = peer.bytes
    t0 = time.perf_counter()
    for _ in range(args.steps):
        m.forward(B)
    ctx.sync()
    elapsed = time.perf_counter() - t0
    res = {"party": party, "elapsed": elapsed, "bytes": ctx.bytes_exchanged, "socket_bytes": peer.bytes - b0,
           "transport": {1: "ipc", 0: "socket"}.get(peer.transport, "none"),
           "out": [int(v) for v in m.output(B)], "key_bytes": len(key) if hasattr(key, "__len__") else None}
    if prof:
        res["prof"] = {k: prof[k] for k in ("aes_calls", "elements", "launches", "hbm_bytes")}
    m.close()
    peer.close()
    ctx.close()
    print(json.dumps(res), flush=True)


def run_party(args):
    """Party mode: the reference's deployment, the two parties as two processes
    on one GPU with their own key and shares, exchanging over a Unix socket
    (gpu_mpc/run_local_2pc.sh:196-233, README.md:99-101).  The two processes are
    started before this process touches the GPU; samples/s = B K / the slower
    party's time for K forwards.  Prints one JSON line."""
    import subprocess
    import tempfile

    import numpy as np

    import synth

    B = args.batch
    dims = synth.Dims(bw=args.bw, slack=args.slack)
    wl = synth.workload(B, dims, seed=args.seed)
    sock = os.path.join(tempfile.mkdtemp(prefix="mpcx_bench_"), "peer.sock")
    base = [sys.executable, os.path.abspath(__file__), "--batch", str(B), "--bw", str(args.bw), "--seed",
            str(args.seed), "--slack", str(args.slack), "--steps", str(args.steps), "--warmup", str(args.warmup),
            "--party-sock", sock]
    log(f"[bench] party mode: starting party 0 and party 1 (B={B}, bw={args.bw}) on {sock}")
    procs = [subprocess.Popen(base + ["--party-child", str(p)], stdout=subprocess.PIPE, text=True) for p in (0, 1)]
    res = []
    try:
        for p in procs:
            o, _ = p.communicate(timeout=900)
            if p.returncode != 0:
                raise RuntimeError(f"party process exited with {p.returncode}")
            res.append(json.loads(o.strip().splitlines()[-1]))
    finally:
        for p in procs:
            if p.poll() is None:
                p.kill()
    elapsed = max(r["elapsed"] for r in res)
    value = B * args.steps / elapsed
    ms_per_step = 1e3 * elapsed / args.steps
    out = np.array(res[0]["out"], np.int64)
    agree = res[0]["out"] == res[1]["out"]
    log(f"[bench] party mode: {args.steps} steps in {elapsed:.3f}s -> {ms_per_step:.2f} ms/step, {value:.1f} samples/s")
    prof = res[0]["prof"]
    step_s = ms_per_step / 1e3
    aes_per_s = prof["aes_calls"] / step_s
    valu_per_aes = (VALU_OPS_PER_AES_MIXED if args.bw == 32 else VALU_OPS_PER_AES)["perm32x2_b512"]
    tops = aes_per_s * valu_per_aes / 1e12
    result = {
        "metric": f"online secure samples/s, party mode (bw={args.bw}, B={B}, 1 GPU, two processes)",
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32" if args.bw == 32 else "u64",
        "data": "synthetic molecules (random trees + ring closures, 10-60 atoms), Kaiming-normal weights",
        "config": {"workload": f"two-party secure affinity forward in party mode: party 0 and party 1 as two "
                               f"processes on one GPU, each with its own key and shares in HBM, exchanging "
                               + ("through device inboxes shared by IPC handles (tokens on a Unix socket)"
                                  if res[0]["transport"] == "ipc" else "over a Unix socket")
                               + f"; bw={args.bw} s=12, B={B} molecules x {dims.n_nodes} atoms, "
                               f"GCN 78-78-156-312, FC 312-1024-128, fusion 256-1024-512-1"
                               + SLACK_DESC.get(args.slack, ""),
                   "B": B, "n_nodes": dims.n_nodes, "bw": args.bw, "scale": dims.s, "lanes": 1,
                   "slack": args.slack, "parties": "two processes", "transport": res[0]["transport"]},
        "bytes_exchanged_per_sample": round(res[0]["bytes"] / args.steps / B, 1),
        "channel_bytes_per_sample": round(res[0]["socket_bytes"] / args.steps / B, 1),
        "channel_equals_counted": all(r["socket_bytes"] == r["bytes"] for r in res),
        "parties_agree": agree,
        "roofline": {
            "kernel": "DCF gate kernels of both parties (k_tr_party_bits / k_tr_party_msg and the one-party "
                      "forms): VALU work of a forward's AES calls over the timed step",
            "bound": "valu",
            "achieved": round(tops, 3),
            "peak": round(VALU_PEAK_TOPS, 2),
            "unit": "TOP/s",
            "frac": round(tops / VALU_PEAK_TOPS, 4),
            "traffic": None,
            "aes_calls_per_step": prof["aes_calls"],
            "valu_ops_per_aes": valu_per_aes,
        },
    }
    try:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import orc
        d = dims
        od = orc.make_dims(bw=d.bw, s=d.s, n_nodes=d.n_nodes, feat=d.feat, gcn=d.gcn, dfc=d.dfc, prot=d.prot,
                           fus=d.fus, lut_nmax=d.lut_nmax, mask_scale=d.mask_scale, slack=d.slack)
        want, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, wl.W)
        result["bit_exact"] = bool(code == 0 and agree and np.array_equal(want, out))
        if not args.no_cpu:
            nb = min(args.cpu_samples, B)
            sl = synth.workload(nb, dims, seed=args.seed)
            k0, k1 = orc.model_keygen(od, nb, 99, sl.W)
            sh = sl.shares
            reps, ct = 0, 0.0
            while ct < args.cpu_seconds or reps == 0:
                t0 = time.perf_counter()
                orc.model_eval(od, nb, sl.W, k0, k1, *sh["x"], *sh["a"], *sh["m"], sl.prot)
                ct += time.perf_counter() - t0
                reps += 1
            result["cpu_baseline"] = {
                "value": round(nb * reps / ct, 3), "unit": "samples/s", **cpu_fields(orc), "kind": "port",
                "sample": f"{reps} x {nb} molecules of the same workload: two-party online eval (both parties in "
                          f"one process, same gates and key format) in oracle/ C with AES-NI + OpenMP, {ct:.1f}s"}
    except Exception as e:
        log(f"[bench] oracle unavailable: {e}")
        result.setdefault("bit_exact", None)
    print(json.dumps(result), flush=True)


def run_shim(args):
    """The reference's whole online path through the drop-in boundary: the
    EzPC-named shim and the sytorch Backend<T> subclasses (include/mpcx_ezpc.hpp,
    include/mpcx_sytorch.hpp) driven by tests/cpp/ezpc_check in the call order of
    ddgSecureAdjNormEval and DeepDTAGenAffinity::_forward (per-sample secret x
    secret matmuls, TrFloor truncations, full-width ReLUs, the mask product, the
    MaskedMaxPoolLayer fold, GPUConcat, FCs, output), the two parties as two
    threads on one channel, both key sets resident in HBM (initGPUKeyArena).
    A step is one forward of both parties (adjacency normalisation included);
    the W + K forwards reuse one key set.  Prints one JSON line."""
    import subprocess
    import tempfile

    import numpy as np

    import synth

    B, bw, S = args.batch, args.bw, 12
    exe = os.path.join(ROOT, "tests", "cpp", "ezpc_check")
    if not os.path.exists(exe):
        raise SystemExit("tests/cpp/ezpc_check is not built (run __graft_entry__.build())")
    dims = synth.Dims(bw=bw)
    wl = synth.workload(B, dims, seed=args.seed)
    N, C = dims.n_nodes, dims.gcn[2]
    T = np.uint32 if bw == 32 else np.uint64
    mod = (1 << bw) - 1

    def ring(v):
        return (np.asarray(v, np.int64).astype(np.uint64) & np.uint64(mod)).astype(T)

    d = tempfile.mkdtemp(prefix="mpcx_shim_")
    maskT = np.repeat((wl.mask << S)[:, :, None], C, axis=2)  # the reference's pre-tiled mask at scale s
    blob, o = [], 0
    for fin, fout in dims.layers():
        blob += [wl.W[o:o + fin * fout], wl.W[o + fin * fout:o + fin * fout + fout] << S]  # bias at scale 2s
        o += fin * fout + fout
    reps = args.warmup + args.steps
    with open(os.path.join(d, "meta.txt"), "w") as f:
        f.write(" ".join(str(v) for v in (bw, B, N, dims.feat, *dims.gcn, *dims.dfc, dims.prot, len(dims.fus),
                                          *dims.fus, S, dims.lut_nmax, reps)) + "\n")
    sh = {"a": wl.shares["a"], "x": wl.shares["x"], "m": synth.share(maskT, bw, args.seed + 50)}
    for k, (s0, s1) in sh.items():
        ring(s0).tofile(os.path.join(d, f"{k}0.bin"))
        ring(s1).tofile(os.path.join(d, f"{k}1.bin"))
    ring(wl.prot).tofile(os.path.join(d, "prot.bin"))
    ring(np.concatenate(blob)).tofile(os.path.join(d, "w.bin"))
    log(f"[bench] shim forward: B={B} bw={bw}, {reps} forwards through ezpc_check")
    r = subprocess.run([exe, "forward", d], capture_output=True, text=True, timeout=1500)
    if r.returncode != 0:
        raise SystemExit(f"ezpc_check forward failed ({r.returncode}): {r.stderr[-2000:]}")
    ms = [float(v) for v in open(os.path.join(d, "time.txt")).read().split()]
    timed = ms[args.warmup:]
    ms_per_step = sum(timed) / len(timed)
    value = B * 1e3 / ms_per_step
    comm = [int(v) for v in open(os.path.join(d, "comm.txt")).read().split()]
    aes = sum(int(v) for v in open(os.path.join(d, "aes.txt")).read().split())
    kb = [int(v) for v in open(os.path.join(d, "keys.txt")).read().split()]
    out = np.fromfile(os.path.join(d, "out.bin"), T).astype(np.int64)
    if bw == 32:
        out = np.where(out >= 1 << 31, out - (1 << 32), out)
    log(f"[bench] shim forward: {ms_per_step:.2f} ms per forward (timed {len(timed)}), {value:.1f} samples/s")
    stats = dict(ln.split() for ln in open(os.path.join(d, "stats.txt")).read().splitlines() if ln.strip())
    log(f"[bench] shim forward, party 0: {stats['rounds']} exchange rounds; backend timers (ms): matmul "
        f"{int(stats['matmul_us']) / 1e3:.2f}, relu {int(stats['relu_us']) / 1e3:.2f}, truncate "
        f"{int(stats['truncate_us']) / 1e3:.2f}")
    valu = VALU_OPS_PER_AES["perm32x2_b512"]
    tops = aes / (ms_per_step / 1e3) * valu / 1e12
    result = {
        "metric": f"online secure samples/s through the EzPC/sytorch drop-in (bw={bw}, B={B}, 1 GPU)",
        "value": round(value, 2),
        "unit": "samples/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u32" if bw == 32 else "u64",
        "data": "synthetic molecules (random trees + ring closures, 10-60 atoms), Kaiming-normal weights",
        "config": {"workload": f"the reference's online path through the drop-in headers: ddgSecureAdjNormEval and "
                               f"DeepDTAGenAffinity::_forward's backend calls (aggregate-first GCN, TrFloor "
                               f"truncations, full-width ReLUs, MaskedMaxPoolLayer), two parties as two threads on "
                               f"one channel, keys resident (initGPUKeyArena); bw={bw} s=12, B={B} molecules x {N} "
                               f"atoms, GCN 78-78-156-312, FC 312-1024-128, fusion 256-1024-512-1",
                   "B": B, "n_nodes": N, "bw": bw, "scale": S},
        "bytes_exchanged_per_sample": round(comm[0] / B, 1),
        "rounds_per_step": int(stats["rounds"]),
        "key_bytes_per_sample_per_party": round(kb[0] / B, 1),
        "roofline": {
            "kernel": "DCF gate evaluation of the shim's gates (both parties): VALU work of a forward's AES calls "
                      "over the timed step",
            "bound": "valu",
            "achieved": round(tops, 3),
            "peak": round(VALU_PEAK_TOPS, 2),
            "unit": "TOP/s",
            "frac": round(tops / VALU_PEAK_TOPS, 4),
            "traffic": None,
            "aes_calls_per_step": aes,
            "valu_ops_per_aes": valu,
        },
    }
    try:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import orc
        od = orc.make_dims(bw=bw, s=S, n_nodes=N, feat=dims.feat, gcn=dims.gcn, dfc=dims.dfc, prot=dims.prot,
                           fus=dims.fus, lut_nmax=dims.lut_nmax, gcn_order=1)
        want, code = orc.plain_forward(od, wl.X, wl.A, wl.mask, wl.prot, wl.W)  # the C++ layers' op order
        result["bit_exact"] = bool(code == 0 and np.array_equal(want, out))
        if not args.no_cpu:
            od.gcn_order = 0
            nb = min(args.cpu_samples, B)
            sl = synth.workload(nb, dims, seed=args.seed)
            k0, k1 = orc.model_keygen(od, nb, 99, sl.W)
            shs = sl.shares
            reps_c, ct = 0, 0.0
            while ct < args.cpu_seconds or reps_c == 0:
                t0 = time.perf_counter()
                orc.model_eval(od, nb, sl.W, k0, k1, *shs["x"], *shs["a"], *shs["m"], sl.prot)
                ct += time.perf_counter() - t0
                reps_c += 1
            result["cpu_baseline"] = {
                "value": round(nb * reps_c / ct, 3), "unit": "samples/s", **cpu_fields(orc), "kind": "port",
                "sample": f"{reps_c} x {nb} molecules of the same workload: the oracle's two-party online eval (both "
                          f"parties, the model's gates and key format) in oracle/ C with AES-NI + OpenMP, {ct:.1f}s"}
    except Exception as e:
        log(f"[bench] oracle unavailable: {e}")
        result.setdefault("bit_exact", None)
    print(json.dumps(result), flush=True)


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import orc
    return orc


def run_copy(args):
    """b = a + 1 over 2^28 int32 on the device (1 GiB read, 1 GiB written per
    step): the plain copy whose FETCH_SIZE / WRITE_SIZE readings scale those
    counters to bytes, and the HBM bandwidth an elementwise kernel reaches."""
    import torch

    n = 1 << 28
    a = torch.ones(n, dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(args.warmup):
        torch.add(a, 1, out=b)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        torch.add(a, 1, out=b)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    assert int(b[0].item()) == 2 and int(b[-1].item()) == 2
    gbs = 2 * 4 * n * args.steps / elapsed / 1e9
    print(json.dumps({
        "metric": "elementwise copy bandwidth (read + write, 1 GPU)", "value": round(gbs, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / max(args.steps, 1), 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int32", "data": "synthetic",
        "config": {"workload": "b = a + 1 over 2^28 int32 (1 GiB read, 1 GiB written per step)"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4)},
    }), flush=True)


def run_relu(args):
    """Secure ReLU over n elements of Z_2^32 (one 31-bit DCF per element and
    party): values uniform in [-8, 8) at scale 12, masked with uniform input
    masks; keys and masked inputs resident in HBM.  One step = one two-party
    evaluation (DCF phase, bit exchange, output shares, reconstruction) of all n
    elements; the reconstruction is checked against max(x, 0)."""
    import ctypes as C

    import numpy as np

    import mpcx

    n, bw, s = args.n, 32, 12
    rng = np.random.default_rng(args.seed)
    x = rng.integers(-8 << s, 8 << s, size=n)
    rin = rng.integers(0, 1 << 32, size=n, dtype=np.uint64)
    ctx = mpcx.Ctx(bw=bw, scale=s)
    if args.aes_variant >= 0:
        ctx.set_aes_variant(args.aes_variant, args.aes_block)
    if args.both_aes >= 0:
        ctx.set_both_party_aes(args.both_aes)
    k0, k1, rout = ctx.tr_keygen(mpcx.RELU, rin, seed=0xACE + args.seed, gate=1)
    key_bytes = int(ctx.lib.mpcx_tr_key_bytes(ctx.h, mpcx.RELU, n))
    dx = mpcx.to_dev(((x.astype(np.uint64) + rin) & 0xFFFFFFFF).astype(np.uint32))
    out = mpcx.empty_dev(4 * n)

    def step():
        ctx.check(ctx.lib.mpcx_tr_eval(ctx.h, mpcx.RELU, n, mpcx.dptr(k0), mpcx.dptr(k1), mpcx.dptr(dx), None, 0,
                                       mpcx.dptr(out)), "tr_eval")

    for _ in range(args.warmup):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    y = mpcx.from_dev(out, np.uint32, n)
    got = ((y.astype(np.int64) - rout.astype(np.int64)) & 0xFFFFFFFF)
    got = np.where(got >= 1 << 31, got - (1 << 32), got)
    exact = bool(np.array_equal(got, np.maximum(x, 0)))
    aes_per_elem = (bw - 1 - 7) + 1  # 31-bit DCF: levels above the 7-level leaf, plus the leaf
    evals = 2.0 * n * args.steps
    aes_s = evals * aes_per_elem / elapsed
    tops = aes_s * VALU_OPS_PER_AES.get(ctx.aes_variant_name(), float("nan")) / 1e12
    # algorithmic HBM bytes per element (both parties): the correction words and
    # leaf once (both parties' threads read party 0's copy), each party's root,
    # mask bit, kappa and G word, the masked input and the revealed output
    per_elem = 16.0 * aes_per_elem + 2.0 * (16.0 + 0.125 + 4.0 + 4.0) + 4.0 + 4.0
    key_gbs = per_elem * n * args.steps / elapsed / 1e9
    result = {
        "metric": "DCF evals/s (secure ReLU, Z_2^32, both parties' evaluations, 1 GPU)",
        "value": round(evals / elapsed, 1),
        "unit": "DCF evals/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(1e3 * elapsed / args.steps, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic: x uniform fixed-point in [-8, 8) at scale 12, uniform masks",
        "config": {"workload": f"secure ReLU microbench, {n} elements, bw=32, keys resident in HBM", "n": n},
        "aes_blocks_per_s": round(aes_s, 1),
        "key_bytes_per_element_per_party": round(key_bytes / n, 2),
        "roofline": {"kernel": "RELU gate call (k_tr_eval)", "bound": "valu",
                     "achieved": round(tops, 3), "peak": round(VALU_PEAK_TOPS, 2), "unit": "TOP/s",
                     "frac": round(tops / VALU_PEAK_TOPS, 4), "co_limit": lds_colimit(aes_s)},
        "roofline_hbm": {"kernel": "k_tr_eval key stream and inputs", "bound": "hbm", "achieved": round(key_gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(key_gbs / HBM_PEAK_GBS, 4)},
        "bit_exact": exact,
    }
    log(f"[relu] {args.steps} x {n} elements in {elapsed:.3f}s: {evals / elapsed / 1e9:.3f} G DCF evals/s")
    if not args.no_cpu:
        try:
            orc = _oracle()
            m = 1 << 16
            ok0, ok1, orout = orc.tr_keygen(7, 1, mpcx.RELU, bw, s, rin[:m])
            xh = (x[:m].astype(np.uint64) + rin[:m]) & 0xFFFFFFFF
            reps, ct = 0, 0.0
            while ct < args.cpu_seconds or reps == 0:
                t0 = time.perf_counter()
                yc, _ = orc.tr_eval(mpcx.RELU, bw, s, ok0, ok1, xh)
                ct += time.perf_counter() - t0
                reps += 1
            gc = (np.asarray(yc, np.int64) - np.asarray(orout, np.int64)) & 0xFFFFFFFF
            gc = np.where(gc >= 1 << 31, gc - (1 << 32), gc)
            result["cpu_baseline"] = {
                "value": round(2.0 * m * reps / ct, 1), "unit": "DCF evals/s", **cpu_fields(orc),
                "kind": "port",
                "sample": f"{reps} x {m} elements of the same workload, both parties, oracle/ C with AES-NI + "
                          f"OpenMP, {ct:.1f}s",
                "bit_exact": bool(np.array_equal(gc, np.maximum(x[:m], 0))),
            }
        except Exception as e:  # the product number stands without the checker
            log(f"[relu] oracle unavailable: {e}")
    print(json.dumps(result), flush=True)
    ctx.close()


def run_adjnorm(args):
    """Secure adjacency normalisation of B=1024 graphs (N=140, Z_2^32): reveal
    A, degrees as row sums of the shares, D^-1/2 through the 8-bit DPF table,
    the outer product T[d_i] T[d_j] (Beaver), one exact truncation, A (.) W
    (Beaver).  Keys and shares resident in HBM; one step = one evaluation of all
    B graphs; the unmasked output is checked against the plaintext formula."""
    import numpy as np

    import mpcx
    import synth

    B, N, bw, nmax = 1024, 140, 32, 138
    _, A, _ = synth.molecules(B, synth.Dims(bw=bw), seed=args.seed + 2)
    a0, a1 = synth.share(A, bw, args.seed + 3)
    ctx = mpcx.Ctx(bw=bw)
    if args.aes_variant >= 0:
        ctx.set_aes_variant(args.aes_variant, args.aes_block)
    if args.both_aes >= 0:
        ctx.set_both_party_aes(args.both_aes)
    ctx.set_adjnorm_lanes(args.lanes)  # concurrent graph groups, each on its own stream
    k0, k1, mask = ctx.adjnorm_keygen(B, N, seed=0xADD + args.seed)
    d0, d1 = mpcx.to_dev(ctx.ring(a0)), mpcx.to_dev(ctx.ring(a1))
    out = mpcx.empty_dev(B * N * N * 4)

    def step():
        ctx.check(ctx.lib.mpcx_adjnorm_eval(ctx.h, B, N, nmax, mpcx.dptr(k0), mpcx.dptr(k1), mpcx.dptr(d0),
                                            mpcx.dptr(d1), mpcx.dptr(out)), "adjnorm_eval")

    for _ in range(args.warmup):
        step()
    ctx.sync()
    ctx.reset_counters()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    ctx.sync()
    elapsed = time.perf_counter() - t0
    P = N * (N + 1) // 2
    got = (mpcx.from_dev(out, np.uint32, B * N * N) - mpcx.from_dev(mask, np.uint32, B * N * N)).astype(np.int64)
    exact = None
    try:
        orc = _oracle()
        exact = bool(np.array_equal(got, orc.adj_norm_plain(A).reshape(-1)))
    except Exception as e:
        log(f"[adjnorm] oracle unavailable: {e}")
    per = elapsed / args.steps
    # AES calls per step: LUT8 (3 per degree and party), TRSLACK (12-bit DCF:
    # 5 levels + leaf per pair and party)
    aes = 2.0 * (3 * B * N + 6 * B * P)
    tops = aes / per * VALU_OPS_PER_AES_MIXED.get(ctx.aes_variant_name(), float("nan")) / 1e12
    result = {
        "metric": "adjacency-normalisation graphs/s (B=1024, N=140, Z_2^32, 1 GPU)",
        "value": round(B / per, 1),
        "unit": "graphs/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(1e3 * per, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u32",
        "data": "synthetic molecular graphs (random trees + ring closures, 10-60 atoms, self loops)",
        "config": {"workload": f"secure adjacency normalisation, B={B} graphs x N={N}, bw=32 s=12, keys resident, "
                               f"{args.lanes} concurrent graph groups",
                   "B": B, "N": N, "lanes": args.lanes},
        "lut_evals_per_s": round(B * N / per, 1),
        "beaver_products_per_s": round(2 * B * N * N / per, 1),
        "truncations_per_s": round(B * P / per, 1),
        "bytes_exchanged_per_graph": round(ctx.bytes_exchanged / (args.steps * B), 1),
        "roofline": {"kernel": "adjacency normalisation call (DCF/DPF AES work over the call)", "bound": "valu",
                     "achieved": round(tops, 3), "peak": round(VALU_PEAK_TOPS, 2), "unit": "TOP/s",
                     "frac": round(tops / VALU_PEAK_TOPS, 4), "co_limit": lds_colimit(aes / per)},
        "bit_exact": exact,
    }
    log(f"[adjnorm] {args.steps} x {B} graphs in {elapsed:.3f}s: {B / per:.0f} graphs/s")
    if not args.no_cpu:
        try:
            orc = _oracle()
            Bs = 16
            ok0, ok1, omask = orc.adjnorm_keygen(bw, 12, Bs, N, 5)
            s0, s1 = a0[:Bs], a1[:Bs]
            reps, ct = 0, 0.0
            while ct < args.cpu_seconds or reps == 0:
                t0 = time.perf_counter()
                oc, _ = orc.adjnorm_eval(bw, 12, Bs, N, nmax, ok0, ok1, s0, s1)
                ct += time.perf_counter() - t0
                reps += 1
            gc = (np.asarray(oc, np.uint64) - np.asarray(omask, np.uint64)) & 0xFFFFFFFF
            result["cpu_baseline"] = {
                "value": round(Bs * reps / ct, 2), "unit": "graphs/s", **cpu_fields(orc), "kind": "port",
                "sample": f"{reps} x {Bs} graphs of the same workload, both parties, oracle/ C with AES-NI + "
                          f"OpenMP, {ct:.1f}s",
                "bit_exact": bool(np.array_equal(gc.astype(np.int64), orc.adj_norm_plain(A[:Bs]).reshape(-1))),
            }
        except Exception as e:  # the product number stands without the checker
            log(f"[adjnorm] oracle unavailable: {e}")
    print(json.dumps(result), flush=True)
    ctx.close()


if __name__ == "__main__":
    main()
