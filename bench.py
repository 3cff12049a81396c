"""Benchmark: 64-bit DCF evaluations per second, 2 parties, N = 2^20, on one
MI355X.

Workload (one step): both parties evaluate their N myl7-format DCF keys
(lambda = 16 bytes, AES-128-MMO PRG, XOR output group, 1-byte payload,
2152 bytes per key) at the public masked inputs xhat_i = x_i + r_in_i, i.e.
2N key evaluations whose XOR reconstructs 1[xhat_i < r_in_i].  Keys and
inputs are resident in HBM before timing starts; keygen runs once on the
device beforehand and is reported separately.

Synthetic inputs (std::mt19937_64 throughout): r_in = mt(1) words;
x = round(N(0,1) * 2^12) by Box-Muller on mt(2); PRG state = low bytes of
mt(3); DCF seeds = bytes of mt(4) words; alpha_i = r_in_i, beta = 0x01.

Prints one JSON line.  --gpus above 1 is refused (single-GPU build).
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "64-bit DCF evals/sec (2 parties, N=2^20) + secure layer latency ms, 1 MI355X"
HBM_PEAK_GBPS = 8000.0
# HBM bytes per dcf_eval_bit_kernel launch at N = 2^20, measured with
# rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE (KiB per dispatch) and scaled by the
# counters' reading for a 256 MiB device copy (FETCH x2.0, WRITE x1.0); the
# commands and raw values are in profiles/dcf_eval_bit_kernel__dcf_batch_n2p20.md.
MEASURED_TRAFFIC_BYTES = 2131324.3 * 1024 * 2.0 + 1200.3 * 1024 * 1.0
# Instructions per dcf_eval_bit_kernel launch at N = 2^20 (rocprofv3 --pmc
# SQ_INSTS_VALU SQ_INSTS_LDS, same profile file): fixed by the compiled kernel
# and N, so lane-ops per second follow from the measured launch time.
DCF_VALU_INSTS = 593684480
DCF_LDS_INSTS = 307299328
VALU_PEAK_GOPS = 256 * 64 * 2.4  # 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, 32-bit integer ops
# LDS: 128 bytes per clock per CU for 4-byte reads (a wave64 ds_read_b32 every
# 2 clocks, random or consecutive addresses alike, measured) x 256 CUs x 2.4 GHz.
LDS_PEAK_GBPS = 256 * 128 * 2.4
INT8_PEAK_TOPS = 5000.0  # dense int8 MFMA, 5.0 POP/s


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--n", type=int, default=1 << 20)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-gates", action="store_true",
                    help="skip the spline-gate and Beaver matmul pipeline timings")
    ap.add_argument("--no-shared", action="store_true",
                    help="configs 2, 4, 5: skip the shared-keystream timings (profiling runs)")
    ap.add_argument("--only", choices=["spline", "matmul", "softmax_ln", "layer", "aes"],
                    help="run one gate pipeline alone and print its result object "
                         "(for profiling; not the benchmark line)")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device-to-device copy kernel 5 times "
                         "(reference point for the FETCH_SIZE / WRITE_SIZE counters)")
    return ap.parse_args()


def calibrate_copy():
    import torch

    n = 256 << 20
    src = torch.empty(n // 8, dtype=torch.int64, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(5):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n, "launches": 5}), flush=True)


def progress(msg):
    """One line per finished stage on stderr (the JSON line stays alone on stdout)."""
    sys.stderr.write("[bench] %s\n" % msg)
    sys.stderr.flush()


def _graph_ms(run, steps, warmup):
    """(ms per run() as one HIP graph replay, ms per eager run()): run()
    issues the whole gate on torch's current stream."""
    import torch

    from suf_amd import tasks

    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        run()
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / steps
    g = tasks.capture(run)
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps, eager_ms


# Device-side spin (core clock cycles, ~0.2-0.4 ms) queued before a start
# event: while it runs the host stages the launch to be timed, so the event
# pair brackets the kernel, not the host's launch overhead on an idle stream.
SPIN_CYCLES = 500_000


def spin():
    import torch

    torch.cuda._sleep(SPIN_CYCLES)


def _launch_ms(run, steps):
    """Mean ms of one launch: events on torch's current stream (the stream
    the launch goes to) right before and after each of `steps` calls, each
    start event behind a device-side spin."""
    import numpy as np
    import torch

    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for s in range(steps):
        spin()
        ev[s][0].record()
        run()
        ev[s][1].record()
    torch.cuda.synchronize()
    return float(np.mean([a.elapsed_time(b) for a, b in ev]))


def roofline_hbm(kernel, kernel_ms, bytes_per_launch, basis, note=None, traffic=None):
    """The contract's roofline object for an HBM-priced kernel: algorithmic
    bytes per launch / the launch's measured mean duration, against 8 TB/s."""
    achieved = bytes_per_launch / (kernel_ms / 1e3) / 1e9
    r = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBPS, "unit": "GB/s",
         "frac": achieved / HBM_PEAK_GBPS, "traffic": traffic, "kernel": kernel,
         "kernel_ms": kernel_ms, "bytes_per_launch": bytes_per_launch, "basis": basis}
    if note:
        r["note"] = note
    return r


def roofline_mfma(kernel, kernel_ms, ops_per_launch, basis, note=None, traffic=None):
    """The same for a matrix-core kernel: int8 MFMA ops per launch / the
    measured launch time, against the dense int8 peak (5.0 POP/s)."""
    achieved = ops_per_launch / (kernel_ms / 1e3) / 1e12
    r = {"bound": "mfma", "achieved": achieved, "peak": INT8_PEAK_TOPS, "unit": "TOP/s (int8)",
         "frac": achieved / INT8_PEAK_TOPS, "traffic": traffic, "kernel": kernel,
         "kernel_ms": kernel_ms, "ops_per_launch": ops_per_launch, "basis": basis}
    if note:
        r["note"] = note
    return r


def cpu_threads():
    """Host threads for the all-cores CPU legs: OMP_NUM_THREADS when set (the
    GPU box sets it to the CPU share of its one GPU), else the CPUs this
    process may run on."""
    v = os.environ.get("OMP_NUM_THREADS", "")
    if v.isdigit() and int(v) > 0:
        return int(v)
    return len(os.sched_getaffinity(0))


def host_info():
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity_cpus": len(os.sched_getaffinity(0)),
            "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"), "cpu_model": model}


def _oracle():
    """The oracle modules (the CPU legs' checker and baseline)."""
    for d in ("tests", "oracle"):
        p = os.path.join(ROOT, d)
        if p not in sys.path:
            sys.path.insert(0, p)
    import fixed_point as fp
    import oracle_lib as ol
    import twoparty_oracle as tp

    ol.aes_use_ni(True)
    return ol, tp, fp


def _timed(fn, threads):
    ol, _, _ = _oracle()
    ol.set_threads(threads)
    try:
        t0 = time.perf_counter()
        r = fn()
        return r, time.perf_counter() - t0
    finally:
        ol.set_threads(0)


# Algorithmic HBM bytes of the two-party task kernels: the streams each
# element (or row) brings in or sends out, both parties.  The truncation
# gates' full-domain tables (2^f entries of which an evaluation reads the
# 16-byte value half) and the LUT blobs are read by every workgroup but
# stay in L2, so they count once per launch, at most 2^f x 16 bytes per gate
# and party.  A CUBIC chain (spline gate, GeLU, nExp) streams x (16), three
# products' triples (3 x 2 parties x 3 words x 8 = 144) and the output (16).
CHAIN_CUBIC_BYTES = 16 + 144 + 16


def trunc_table_bytes(gates, f=12):
    """Bytes of the value halves of `gates` truncation tables, both parties."""
    return gates * 2 * (1 << f) * 16


def softmax_bytes(n_packed, rows, pre=0, indexed_input=False, out_written=True, n_dense=0,
                  dense_planes=False):
    """The softmax block kernels' streams: per packed element the scores (16, + a
    4-byte index), the nExp chain's triples (144), the normalisation's a and
    c shares (32), the probabilities (16); per row the reciprocal chain's
    triples (144), the normalisation's b shares (16) and the row offset (4);
    per dense element the A shares (16) and the open (8, + 8 for its digit
    planes); once per launch the tables of the `pre` score truncations, the
    nExp and reciprocal chains' three gates each and the normalisation's."""
    per = 16 + (4 if indexed_input else 0) + 144 + 32 + (16 if out_written else 0)
    return (n_packed * per + rows * (144 + 16 + 4)
            + n_dense * (16 + 8 + (8 if dense_planes else 0))
            + trunc_table_bytes(pre + 3 + 3 + 1))


# HBM traffic per launch of the config 2-5 kernels at the default shapes with
# per-party keystreams: rocprofv3 --pmc FETCH_SIZE, then WRITE_SIZE (KiB per
# dispatch, mean over the run's launches of the kernel), scaled by the
# counters' reading for a 256 MiB device copy (FETCH x2.0, WRITE x1.0); the
# commands and raw values are in profiles/per_party_keystreams__spline_n2p20__
# softmax_ln__secure_layer.md (the matmul product's in profiles/gate_pipelines__
# spline_n2p20__matmul_128x768x3072__softmax_ln.md).
def _traffic(fetch_kib, write_kib):
    if fetch_kib is None or write_kib is None:
        return None
    return fetch_kib * 1024 * 2.0 + write_kib * 1024 * 1.0


SPLINE_CHAIN_TRAFFIC = _traffic(85280.0, 16384.0)
MATMUL_PRODUCT_TRAFFIC = _traffic(41173, 6144)
SOFTMAX_TRAFFIC = _traffic(14919.3, 1560.0)
LAYER_SOFTMAX_TRAFFIC = _traffic(17666.4, 4616.1)


def bench_spline(steps, warmup, n=1 << 20, frac_bits=12, cpu_seconds=0.0, shared=True):
    """The spline gate (interval LUT + three Beaver products + GapARS by f and
    2f) for both parties on N = 2^20 inputs x = clip(3 N(0,1), +-8) in Q12
    (Box-Muller on mt(5)); coefficients from mt(6); dealer randomness mt(7).
    Returns ms per gate evaluation (both parties), the chain kernel's roofline
    and, with cpu_seconds > 0, the CPU baseline and the reconstruction check."""
    import numpy as np
    import torch

    from suf_amd import pfss, spline, tasks

    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    alpha, coeffs = spline.spline_spec(frac_bits, seed=6)
    x = pfss.host_normal_fixed(5, 3.0, 8.0, frac_bits, n)
    x0 = pfss.host_mt19937_64(8, n)
    x1 = (x - x0).astype(np.uint64)
    gate = spline.SplineGate(n, alpha, coeffs, state, frac_bits, seed=7)
    xd = [torch.from_numpy(v.view(np.int64).copy()).cuda() for v in (x0, x1)]
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]

    def run():
        # The truncations' key-only halves first, on the same stream.
        gate.eval2(xd, out, prep=(tasks.Prepared(None, [gate.truncs()]), 0))

    # The chain launch alone (its truncations prepared once beforehand).
    prepared = tasks.Prepared(None, [gate.truncs()])
    chain = lambda: gate.eval2(xd, out, prep=(prepared, 0))  # noqa: E731
    with pfss.keystream_per_party():
        ms, eager_ms = _graph_ms(run, steps, warmup)
        chain()
        chain_ms = _launch_ms(chain, steps)
    gpu = [out[0].cpu().numpy().view(np.uint64).copy(), out[1].cpu().numpy().view(np.uint64).copy()]
    # The same with one keystream for both parties (one process, one dealer key).
    ms_shared = chain_ms_shared = None
    if shared:
        ms_shared, _ = _graph_ms(run, steps, warmup)
        chain()
        chain_ms_shared = _launch_ms(chain, steps)
    nbytes = CHAIN_CUBIC_BYTES * n + trunc_table_bytes(3, frac_bits)
    res = {"ms": ms, "eager_ms": eager_ms, "n": n, "frac_bits": frac_bits,
           "intervals": int(gate.intervals),
           "trunc": "GapARS f=%d (x3: the 2f truncation as two f truncations)" % frac_bits,
           "steps": steps,
           "roofline": roofline_hbm("gate_chain_kernel (CUBIC)", chain_ms, nbytes,
                                    "%d B per element (x 16, triples 144, out 16) x N + 3 "
                                    "truncation tables once (2 x 2^%d x 16 B each)"
                                    % (CHAIN_CUBIC_BYTES, frac_bits),
                                    note="per-party keystreams; the chain's AES-CTR keystream "
                                         "and dependent steps bind it, not HBM",
                                    traffic=SPLINE_CHAIN_TRAFFIC if n == 1 << 20 else None),
           "keystream": "per party",
           "ms_shared": ms_shared, "chain_ms_shared": chain_ms_shared,
           "keystream_note": "ms and the roofline: each party computes its own LUT keystream, "
                             "as two parties in separate processes do.  Both parties' blobs come "
                             "from one dealer key (seed_from_id), so one process can compute each "
                             "keystream block once for both: *_shared",
           "check": "not run (--no-cpu)"}
    if cpu_seconds > 0:
        res.update(cpu_spline_baseline(gate, state, x, x0, x1, gpu, alpha, coeffs, frac_bits))
    return res


def cpu_spline_baseline(gate, state, x, x0, x1, gpu, alpha, coeffs, f):
    """The same two-party spline gate on the host: the oracle's composition of
    the protocol steps (interval LUT, Beaver products, truncation gates with
    their DCF walks), one C call per step over the whole batch, OpenMP on all
    host threads; then one thread on the first 2^14 elements.  Shares compared
    with the GPU's, reconstruction checked against the closed form."""
    import numpy as np

    ol, tp, fp = _oracle()
    n = x0.size
    T = cpu_threads()
    got, dt = _timed(lambda: tp.spline2(ol.Prg(state), gate, (x0, x1)), T)
    mism = sum(int(np.count_nonzero(got[p] != gpu[p])) for p in (0, 1))
    m1 = min(n, 1 << 14)
    sl = slice(0, m1)
    _, dt1 = _timed(lambda: tp.spline2(ol.Prg(state), gate, (x0[sl], x1[sl]), sl=sl), 1)
    rec = (gpu[0] + gpu[1]).astype(np.uint64)
    ok = bool(np.array_equal(rec, fp.spline_closed_form(alpha, coeffs, x, f))) and mism == 0
    return {"check": "ok" if ok else "MISMATCH",
            "cpu_baseline": {"value": dt * 1e3, "unit": "ms per gate (both parties, N=2^20)",
                             "cores": T, "kind": "port",
                             "ms_1thread": dt1 * 1e3 * n / m1,
                             "sample": "all %d elements on %d threads (oracle composition of the "
                                       "LUT, Beaver and truncation-gate steps, one C call per step, "
                                       "AES instructions); ms_1thread: the first %d elements on one "
                                       "thread, scaled to N; shares compared with the GPU: %d "
                                       "mismatches" % (n, T, m1, mism),
                             "mismatches": mism, "host": host_info()}}


def bench_matmul(steps, warmup, M=128, K=768, N=3072, frac_bits=12, cpu_seconds=0.0):
    """Beaver matmul + GapARS truncation for both parties: X [128 x 768] =
    round(N(0,1) 2^12) (mt(8)), W [768 x 3072] = round(N(0,0.02) 2^12) (mt(9)),
    both additively shared (mt(108), mt(109)); triples and truncation key from
    mt(10), mt(11).  Returns ms per evaluation, the product kernel's roofline
    and the reconstruction check."""
    import numpy as np
    import torch

    from suf_amd import matmul_gate, pfss

    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    X = pfss.host_normal_fixed(8, 1.0, 0.0, frac_bits, M * K)
    W = pfss.host_normal_fixed(9, 0.02, 0.0, frac_bits, K * N)
    X0, W0 = pfss.host_mt19937_64(108, M * K), pfss.host_mt19937_64(109, K * N)
    dev = lambda v: torch.from_numpy(np.ascontiguousarray(v).view(np.int64).copy()).cuda()
    Xd = [dev(X0), dev((X - X0).astype(np.uint64))]
    Wd = [dev(W0), dev((W - W0).astype(np.uint64))]
    g = matmul_gate.BeaverMatmulTrunc(M, K, N, state, frac_bits, seed=10)
    out = [torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2)]
    for _ in range(warmup):
        g.eval2(Xd, Wd, out)
    torch.cuda.synchronize()
    # The opens-as-planes launch and the product launch, eager, with events
    # between them; then the whole gate as one graph replay.
    nev = 3 if g.fused else 2
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(nev)] for _ in range(steps)]
    for s in range(steps):
        g.eval2(Xd, Wd, out, events=ev[s])
    torch.cuda.synchronize()
    mm_ms = float(np.mean([e[0].elapsed_time(e[-1]) for e in ev]))
    prod_ms = float(np.mean([e[-2].elapsed_time(e[-1]) for e in ev]))
    ms, eager_ms = _graph_ms(lambda: g.eval2(Xd, Wd, out), steps, warmup)
    prod = X.view(np.int64).reshape(M, K) @ W.view(np.int64).reshape(K, N)
    rec = (out[0].cpu().numpy().view(np.uint64) + out[1].cpu().numpy().view(np.uint64))
    ok = bool(np.array_equal(rec.astype(np.uint64), (prod >> frac_bits).view(np.uint64).ravel()))
    macs = 2 * 2 * M * K * N  # both parties, [D | A] x [B' ; E] is a 2K-deep product
    res = {"ms": ms, "eager_ms": eager_ms, "shape": [M, K, N], "matmul_ms": mm_ms,
           "matmul_part": ("opens written as digit planes + both products + truncation "
                           "(eager, events around them)" if g.fused else
                           "both products (eager, events around them)"),
           "u64_macs": macs,
           "u64_mac_per_s": macs / (mm_ms / 1e3), "trunc": "GapARS f=%d" % frac_bits,
           "matmul_kernel": ("two-party int8-digit MFMA, truncation fused" if g.fused else
                             "int8-limb MFMA" if g.mm_work is not None else "u64 VALU"),
           "steps": steps, "check": "ok" if ok else "MISMATCH"}
    if g.fused:
        # Per 32 x 32 tile and 32-deep k-step each party runs 2 x 36
        # digit-plane MFMAs (party 0: (D + A0) E and D B0; party 1: A1 E and
        # D B1); each is 32x32x32 int8 MACs.
        mfmas = (M // 32) * (N // 32) * (K // 32) * (72 + 72)
        res["product_ms"] = prod_ms
        res["roofline"] = roofline_mfma(
            "beaver_bal_kernel", prod_ms, mfmas * 2 * 32 * 32 * 32,
            "%d v_mfma_i32_32x32x32_i8 (tiles x k-steps x 144 digit products) x 65536 ops" % mfmas,
            traffic=MATMUL_PRODUCT_TRAFFIC if (M, K, N) == (128, 768, 3072) else None)
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_matmul_baseline(g, state, Xd, Wd, out, cpu_seconds)
    return res


def cpu_matmul_baseline(g, state, Xd, Wd, out, seconds):
    """Beaver matmul + truncation on the host: the oracle's OpenMP u64 matmul
    (src/nn/matmul_beaver.cpp:139-161 semantics and loop order) for both
    parties and the oracle truncation gate, 8 rows at a time until every row
    is done or the time budget is used, on all host threads; then 8 rows on
    one thread.  Outputs compared with the GPU's."""
    import numpy as np

    ol, _, _ = _oracle()
    T = cpu_threads()
    M, K, N, f = g.M, g.K, g.N, g.f
    h = lambda t: t.cpu().numpy().view(np.uint64)
    X = [h(Xd[0]).reshape(M, K), h(Xd[1]).reshape(M, K)]
    W = [h(Wd[0]), h(Wd[1])]
    A = [h(a).reshape(M, K) for a in g.A]
    B = [h(b) for b in g.B]
    C = [h(c).reshape(M, N) for c in g.C]
    keys = [k.cpu().numpy() for k in g.keys]
    gpu = [h(o).reshape(M, N) for o in out]
    prg = ol.Prg(state)
    E = ((W[0] - B[0]) + (W[1] - B[1])).astype(np.uint64)
    rin = sum(g.rin) & ((1 << 64) - 1)

    def rows_block(r, threads):
        D = ((X[0][r] - A[0][r]) + (X[1][r] - A[1][r])).astype(np.uint64)
        nr = D.shape[0]
        Z = [ol.beaver_matmul(p, D, E, A[p][r], B[p], C[p][r], 1, nr, K, N, threads=threads)
             for p in (0, 1)]
        zhat = (Z[0] + Z[1] + np.uint64(rin)).astype(np.uint64)
        return [ol.trunc_eval(prg, ol.TRUNC_GAPARS, f, keys[p], zhat) for p in (0, 1)]

    rows, mism = 0, 0
    ol.set_threads(T)
    t0 = time.perf_counter()
    while rows + 8 <= M:
        r = slice(rows, rows + 8)
        y = rows_block(r, T)
        mism += sum(int(np.count_nonzero(y[p] != gpu[p][r].ravel())) for p in (0, 1))
        rows += 8
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    ol.set_threads(1)
    t1 = time.perf_counter()
    rows_block(slice(0, 8), 1)
    dt1 = time.perf_counter() - t1
    ol.set_threads(0)
    macs = 2 * 2 * rows * K * N
    return {"value": macs / dt, "unit": "u64 MAC/s (both parties, with truncation)",
            "cores": T, "kind": "port", "ms_full_shape": dt * M / rows * 1e3,
            "ms_full_shape_1thread": dt1 * M / 8 * 1e3,
            "sample": "%d of the %d output rows on %d threads (oracle C matmul with the "
                      "reference's loop order, then the oracle truncation gate); 1 thread: 8 "
                      "rows, scaled; outputs compared with the GPU: %d mismatches"
                      % (rows, M, T, mism), "mismatches": mism, "host": host_info()}


def bench_softmax_ln(steps, warmup, frac_bits=12, cpu=True, shared=True):
    """Softmax over 12 heads x 128 x 128 causal score rows (scores
    round(N(0,2) 2^12), mt(11)) followed by LayerNorm over 128 x 768
    (round(N(0,1) 2^12), mt(12)), both parties; shares from mt(111), mt(121);
    dealer material from suf_amd.tasks.Dealer(11), Dealer(12).  Returns ms
    per block (softmax + LayerNorm), each part, and the softmax kernel's
    roofline."""
    import numpy as np
    import torch

    from suf_amd import layernorm, pfss, softmax

    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    offs = softmax.causal_offsets(12, 128)
    n_sm = int(offs[-1])
    rows, cols = 128, 768
    sc = pfss.host_normal_fixed(11, 2.0, 0.0, frac_bits, n_sm)
    xl = pfss.host_normal_fixed(12, 1.0, 0.0, frac_bits, rows * cols)
    dev = lambda v: torch.from_numpy(np.ascontiguousarray(v).view(np.int64).copy()).cuda()

    def shares(v, seed):
        v0 = pfss.host_mt19937_64(seed, v.size)
        return v0, (v - v0).astype(np.uint64)

    s0, s1 = shares(sc, 111)
    l0, l1 = shares(xl, 121)
    sin, lin = (dev(s0), dev(s1)), (dev(l0), dev(l1))
    sm = softmax.SoftmaxBlock(offs, state, frac_bits, seed=11)
    ln = layernorm.LayerNormBlock(rows, cols, state, frac_bits, seed=12)
    sout = tuple(torch.empty(n_sm, dtype=torch.int64, device="cuda") for _ in range(2))
    lout = tuple(torch.empty(rows * cols, dtype=torch.int64, device="cuda") for _ in range(2))
    from suf_amd import tasks

    def run(ev=None):
        # Both blocks' truncation key-only halves in one batched walk first,
        # on the same stream; then the two one-launch blocks.
        prep = (tasks.Prepared(None, [sm.truncs() + ln.truncs()]), 0)
        if ev:
            spin()
            ev[0].record()
        sm.eval2(sin, sout, prep=prep)
        if ev:
            ev[1].record()
            spin()
            ev[2].record()
        ln.eval2(lin, lout, prep=prep)
        if ev:
            ev[3].record()

    def split_ms():
        ev = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(steps)]
        for s in range(steps):
            run(ev[s])
        torch.cuda.synchronize()
        return (float(np.mean([e[0].elapsed_time(e[1]) for e in ev])),
                float(np.mean([e[2].elapsed_time(e[3]) for e in ev])))

    with pfss.keystream_per_party():
        ms, eager_ms = _graph_ms(run, steps, warmup)
        sm_ms, ln_ms = split_ms()
    gpu_s = [sout[p].cpu().numpy().view(np.uint64).copy() for p in (0, 1)]
    gpu_l = [lout[p].cpu().numpy().view(np.uint64).copy() for p in (0, 1)]
    ms_shared = sm_ms_shared = ln_ms_shared = None
    if shared:
        ms_shared, _ = _graph_ms(run, steps, 1)
        sm_ms_shared, ln_ms_shared = split_ms()
    res = {"ms": ms, "eager_ms": eager_ms, "softmax_ms": sm_ms, "layernorm_ms": ln_ms,
           "split": "softmax_ms / layernorm_ms: each block's one launch, eager, without the "
                    "shared prepare walk",
           "softmax_shape": "12 heads x 128 causal rows (%d scores)" % n_sm,
           "layernorm_shape": [rows, cols], "frac_bits": frac_bits, "steps": steps,
           "roofline": roofline_hbm(
               "softmax2_team_kernel", sm_ms, softmax_bytes(n_sm, len(offs) - 1),
               "per score 16 in + nExp triples 144 + normalisation shares 32 + 16 out; per row "
               "164; 7 truncation tables once (2 x 2^12 x 16 B each)",
               note="per-party keystreams; bound by each row's chain of dependent steps (max "
                    "tree rounds, keystream AES, table reads), not HBM",
               traffic=SOFTMAX_TRAFFIC),
           "layernorm_bytes": rows * cols * (16 + 48 + 32 + 16),
           "keystream": "per party",
           "ms_shared": ms_shared, "softmax_ms_shared": sm_ms_shared,
           "layernorm_ms_shared": ln_ms_shared,
           "keystream_note": "ms, the split and the roofline: each party computes its own LUT "
                             "keystreams; *_shared: one keystream block for both parties (one "
                             "process, one dealer key per gate)",
           "check": "not run (--no-cpu)"}
    if cpu:
        res.update(cpu_softmax_ln_baseline(state, sm, ln, (s0, s1), (l0, l1), sc, xl, gpu_s,
                                           gpu_l, frac_bits))
    return res


def cpu_softmax_ln_baseline(state, sm, ln, sx, lx, sc, xl, gpu_s, gpu_l, f):
    """The same two-party softmax and LayerNorm chains on the host, composed
    from the oracle's steps (interval LUT, Beaver, truncation gate with its DCF
    walks), one C call per step over the whole block, on all host threads and
    on one; shares compared with the GPU's, reconstruction checked against
    the fixed-point closed form."""
    import numpy as np

    ol, tp, fp = _oracle()
    T = cpu_threads()

    def both():
        t0 = time.perf_counter()
        prob, _ = tp.softmax2(ol.Prg(state), sm, list(sx))
        t1 = time.perf_counter()
        y = tp.layernorm2(ol.Prg(state), ln, list(lx))
        return prob, y, t1 - t0, time.perf_counter() - t1

    (prob, y, tsm, tln), dt = _timed(both, T)
    (_, _, tsm1, tln1), dt1 = _timed(both, 1)
    mism = sum(int(np.count_nonzero(prob[p] != gpu_s[p])) for p in (0, 1))
    mism += sum(int(np.count_nonzero(y[p] != gpu_l[p])) for p in (0, 1))
    want_p, _ = fp.softmax_block(sc, sm.offsets, sm.nexp_table, sm.recip.table, f)
    want_y, _ = fp.layernorm(xl, ln.rows, ln.cols, f, ln.inv_len, ln.eps_q, ln.rsqrt.table)
    rec_ok = (np.array_equal((gpu_s[0] + gpu_s[1]).astype(np.uint64), want_p.view(np.uint64))
              and np.array_equal((gpu_l[0] + gpu_l[1]).astype(np.uint64),
                                 want_y.view(np.uint64)))
    return {"check": "ok" if rec_ok and mism == 0 else "MISMATCH",
            "cpu_baseline": {"value": dt * 1e3, "unit": "ms per block (both parties)",
                             "softmax_ms": tsm * 1e3, "layernorm_ms": tln * 1e3,
                             "cores": T, "kind": "port", "ms_1thread": dt1 * 1e3,
                             "softmax_ms_1thread": tsm1 * 1e3, "layernorm_ms_1thread": tln1 * 1e3,
                             "sample": "the whole block on %d threads and on one (oracle "
                                       "composition of the LUT, Beaver and truncation-gate "
                                       "steps, one C call per step); shares compared with the "
                                       "GPU: %d mismatches" % (T, mism),
                             "mismatches": mism, "host": host_info()}}


LAYER_DEVIATIONS = [
    "driven by suf_amd/layer.py (the task chains as launches), not by SUF's PhaseExecutor",
    "every truncation gate has its own key (the reference shares one per task)",
    "2f truncations (scores, variance, CubicPolyTask's last step) run as two f-bit gates "
    "(the same floor)",
    "rsqrt's halving is one truncation by f+1 (ref_rsqrt_fixed's value)",
    "the score scale inv_sqrt is a public factor inside the truncation's open (the reference "
    "scales each share in the matmul epilogue: the same value up to one unit before the shift)",
    "one Beaver triple per head for the attention products",
    "64-bit ring (the reference GPT-2 bench uses 50 bits)",
]


def bench_layer(steps, warmup, frac_bits=12, cpu=True, shared=True):
    """One GPT-2-small-shaped secure layer (hidden 768, 12 heads, seq 128, FFN
    3072, GeLU) for both parties: weights round(N(0,0.02) 2^12) (mt(13) and
    derived seeds), input x = round(N(0,1) 2^12) (mt(14)) shared with mt(141);
    dealer material from suf_amd.tasks.Dealer(13).  Times the whole layer as
    one HIP graph replay (and eagerly, with a per-stage breakdown)."""
    import numpy as np
    import torch

    from suf_amd import layer, pfss, tasks

    seq, d, heads, ffn = 128, 768, 12, 3072
    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    W = layer.synthetic_weights(d, ffn, frac_bits, 13)
    x = pfss.host_normal_fixed(14, 1.0, 0.0, frac_bits, seq * d)
    x0 = pfss.host_mt19937_64(141, seq * d)
    x1 = (x - x0).astype(np.uint64)
    dev = lambda v: torch.from_numpy(np.ascontiguousarray(v).view(np.int64).copy()).cuda()
    xin = (dev(x0), dev(x1))
    ly = layer.TransformerLayer(state, W, seq, d, heads, ffn, frac_bits, seed=13)
    out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn):
        e0.record()
        for _ in range(steps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    def measure():
        """(graph ms, eager ms, per-stage eager ms, softmax launch ms, graph,
        eager outputs, replays match) under the current keystream policy."""
        for _ in range(warmup):
            ly.eval2(xin, out)
        torch.cuda.synchronize()
        eager_ms = timed(lambda: ly.eval2(xin, out))
        # Per-stage split of one more eager run (events between stages;
        # launch overhead included, so the stages sum to more than the graph
        # replay), and the softmax block's launch in each eager run.
        stages = ["ln1", "qkv", "attention", "out_proj+residual", "ln2", "w1", "gelu",
                  "w2+residual"]
        m = []
        ly.eval2(xin, out, marks=m)
        torch.cuda.synchronize()
        per_stage = {stages[i]: m[i].elapsed_time(m[i + 1]) for i in range(len(stages))}
        smk = []
        for _ in range(steps):
            ly.eval2(xin, out, sm_marks=smk, sm_spin=spin)
        torch.cuda.synchronize()
        sm_ms = float(np.mean([smk[2 * i].elapsed_time(smk[2 * i + 1])
                               for i in range(len(smk) // 2)]))
        eager_out = [out[0].cpu().numpy().view(np.uint64).copy(),
                     out[1].cpu().numpy().view(np.uint64).copy()]
        g = tasks.capture(lambda: ly.eval2(xin, out))
        torch.cuda.synchronize()
        ok = True
        for _ in range(2):  # replays agree with the eager result
            g.replay()
            torch.cuda.synchronize()
            ok = ok and all(np.array_equal(out[p].cpu().numpy().view(np.uint64), eager_out[p])
                            for p in (0, 1))
        return timed(g.replay), eager_ms, per_stage, sm_ms, g, eager_out, ok

    with pfss.keystream_per_party():
        graph_ms, eager_ms, per_stage, sm_ms, g, eager_out, replay_ok = measure()
    graph_ms_shared = eager_ms_shared = sm_ms_shared = None
    if shared:
        graph_ms_shared, eager_ms_shared, _, sm_ms_shared, _, eager_shared, ok_shared = measure()
        replay_ok = replay_ok and ok_shared and all(
            np.array_equal(eager_out[p], eager_shared[p]) for p in (0, 1))
    at = ly.attn
    res = {"ms": graph_ms, "eager_ms": eager_ms, "stages_eager_ms": per_stage,
           "shape": {"seq": seq, "hidden": d, "heads": heads, "ffn": ffn}, "frac_bits": frac_bits,
           "ring": "Z_2^64", "steps": steps, "graph_replays_match_eager": replay_ok,
           "roofline": roofline_hbm(
               "softmax2_team_kernel (scores' two truncations, softmax, open of P - A as planes)",
               sm_ms, softmax_bytes(at.n, heads * seq, pre=2, indexed_input=True,
                                    out_written=False, n_dense=heads * seq * seq,
                                    dense_planes=True),
               "per packed score 20 in + nExp triples 144 + normalisation shares 32; per row "
               "164; per dense entry 32; 9 truncation tables once (2 x 2^12 x 16 B each)",
               note="per-party keystreams; the layer's largest kernel, bound by each row's "
                    "dependent chain",
               traffic=LAYER_SOFTMAX_TRAFFIC),
           "keystream": "per party",
           "ms_shared": graph_ms_shared, "eager_ms_shared": eager_ms_shared,
           "softmax_ms_shared": sm_ms_shared,
           "keystream_note": "ms, the stages and the roofline: each party computes its own LUT "
                             "keystreams, as two parties in separate processes do; *_shared: "
                             "one keystream block for both parties (one process, one dealer key "
                             "per gate); both policies give the same shares",
           "protocol_deviations": LAYER_DEVIATIONS,
           "check": "not run (--no-cpu)" if replay_ok else "MISMATCH"}
    if cpu:
        res.update(cpu_layer_baseline(state, ly, x, x0, x1, W, eager_out, replay_ok, frac_bits))
    return res


def cpu_layer_baseline(state, ly, x, x0, x1, W, gpu, replay_ok, f):
    """The same two-party layer on the host: the oracle's composition of every
    protocol step of suf_amd/layer.py (LayerNorm, public products with their
    truncation gates, per-head Beaver products, softmax, GeLU), one C call per
    step, on all host threads and on one; shares compared with the GPU's, the
    reconstruction checked against the fixed-point closed form."""
    import numpy as np

    ol, tp, fp = _oracle()
    from suf_amd import tables

    T = cpu_threads()
    (y, _), dt = _timed(lambda: tp.layer2(ol.Prg(state), ly, (x0, x1)), T)
    _, dt1 = _timed(lambda: tp.layer2(ol.Prg(state), ly, (x0, x1)), 1)
    mism = sum(int(np.count_nonzero(y[p] != gpu[p])) for p in (0, 1))
    tabs = {"nexp": tables.nexp_table(f), "recip": tables.recip_table(f),
            "rsqrt": tables.rsqrt_table(f), "gelu": tables.gelu_table(f)}
    t0 = time.perf_counter()
    want, _ = fp.transformer_layer(x, W, ly.seq, ly.d, ly.heads, ly.ffn, f, tabs,
                                   tables.inv_len_qf(ly.d), tables.eps_qf())
    cf = time.perf_counter() - t0
    rec = (gpu[0] + gpu[1]).astype(np.uint64)
    ok = replay_ok and mism == 0 and bool(np.array_equal(rec, want.view(np.uint64)))
    return {"check": "ok" if ok else "MISMATCH", "closed_form_cpu_ms": cf * 1e3,
            "cpu_baseline": {"value": dt * 1e3, "unit": "ms per layer (both parties)",
                             "cores": T, "kind": "port", "ms_1thread": dt1 * 1e3,
                             "sample": "the whole layer on %d threads and on one (oracle "
                                       "composition of every protocol step: LayerNorm, public "
                                       "products, truncation gates, per-head Beaver products, "
                                       "softmax, GeLU; one C call per step); shares compared "
                                       "with the GPU: %d mismatches" % (T, mism),
                             "mismatches": mism, "host": host_info()}}


def cpu_baseline(keys0, keys1, xhat, gpu_bits0, gpu_bits1, seconds):
    """The oracle's restatement of the myl7 batch evaluation (dcf.c:146-193
    walked per key, Myl7FssBackend::eval_dcf_many_u64 semantics,
    include/proto/myl7_fss_backend.hpp:73-100) with the AES instructions and
    OpenMP over keys: all host threads, then one thread, each over the same
    sample of keys for half of the time budget."""
    import numpy as np

    ol, _, _ = _oracle()
    state = ol.mt64_bytes(3, 128)
    prg = ol.Prg(state.tobytes())
    n = keys0.shape[0]
    mism = [0]

    def run(threads, budget):
        done = 0
        t0 = time.perf_counter()
        while True:
            for keys, gb in ((keys0, gpu_bits0), (keys1, gpu_bits1)):
                o = ol.myl7_eval_many_bit(prg, 0, 64, keys, xhat, threads=threads)
                mism[0] += int(np.count_nonzero(o != gb))
                done += n
            if time.perf_counter() - t0 >= budget:
                break
        return done, time.perf_counter() - t0

    T = cpu_threads()
    done, dt = run(T, seconds / 2)
    m1 = min(n, 1 << 13)
    k0, k1, x1s = keys0, keys1, xhat
    keys0, keys1, xhat = k0[:m1], k1[:m1], x1s[:m1]
    gpu_bits0, gpu_bits1 = gpu_bits0[:m1], gpu_bits1[:m1]
    n = m1
    done1, dt1 = run(1, seconds / 2)
    return {
        "value": done / dt,
        "unit": "evals/s",
        "cores": T,
        "kind": "port",
        "value_1thread": done1 / dt1,
        "aes": "x86 AES instructions" if ol.LIB.orc_aes_ni_active() else "FIPS-197 table-free",
        "sample": "%d DCF evals on %d threads over the first %d keys per party of the same N=2^20 "
                  "batch (cycled), and %d on one thread over the first %d; the oracle's myl7 "
                  "dcf_eval restatement (4 AES per level as dcf.c) with OpenMP over keys; shares "
                  "compared with the GPU: %d mismatches"
                  % (done, T, k0.shape[0], done1, m1, mism[0]),
        "mismatches": mism[0],
        "host": host_info(),
    }


def cpu_baseline_reference(keys0, keys1, xhat, gpu_bits0, gpu_bits1, seconds):
    """The reference's own CPU backend on the same keys: Myl7FssBackend::
    eval_dcf_many_u64 (include/proto/myl7_fss_backend.hpp:73-100, a serial
    loop over keys; dcf.c and aes128_mmo.c with OpenSSL EVP AES) compiled from
    the reference sources by oracle/build_ref.sh into oracle/_ref.  One
    thread, as the reference's batch loop runs; keys cycled for the time
    budget; shares compared with the GPU's.  None where that build is absent."""
    import numpy as np

    ol, _, _ = _oracle()
    if not ol.ref_available(ol.GROUP_XOR):
        return None
    ref = ol.ref_lib(ol.GROUP_XOR)
    state = ol.mt64_bytes(3, 128)
    ref.ref_prg_init(ol.ptr(state), ol.PRG_STATE_BYTES)
    n, kb = keys0.shape
    xs = np.ascontiguousarray(xhat[:n], dtype=np.uint64)
    out = np.zeros(n, dtype=np.uint8)
    done, mism = 0, 0
    t0 = time.perf_counter()
    while True:
        for keys, gb in ((keys0, gpu_bits0), (keys1, gpu_bits1)):
            flat = np.ascontiguousarray(keys)
            rc = ref.ref_adapter_eval_many(64, kb, ol.ptr(flat), ol.ptr(xs, ol.u64p), n, 1,
                                           ol.ptr(out))
            if rc != 0:
                return None
            mism += int(np.count_nonzero(out != gb[:n]))
            done += n
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "evals/s", "cores": 1, "kind": "reference",
            "sample": "%d DCF evals over the first %d keys per party of the same N=2^20 batch "
                      "(cycled): the reference's Myl7FssBackend::eval_dcf_many_u64 built from "
                      "its own sources (oracle/build_ref.sh), one thread as its batch loop; "
                      "shares compared with the GPU: %d mismatches" % (done, n, mism),
            "mismatches": mism, "host": host_info()}


def bench_aes(steps, warmup, blocks=1 << 24):
    """AES-128-CTR keystream of `blocks` blocks by the LDS T-table kernel and
    by the bitsliced one (the alternative the DCF's AES was chosen against):
    launch times by events behind a device-side spin, blocks per second, and
    the two outputs compared with each other (the GPU tests compare each form
    with the oracle)."""
    import numpy as np
    import torch

    from suf_amd import pfss

    rk = bytes(range(176))
    outs = {k: torch.empty(blocks * 16, dtype=torch.uint8, device="cuda")
            for k in ("ttable", "bitsliced")}
    res = {"blocks": blocks}
    for name in ("ttable", "bitsliced"):
        bs = name == "bitsliced"
        for _ in range(warmup):
            pfss.aes128_ctr(rk, 5, 7, blocks, bitsliced=bs, out=outs[name])
        ms = []
        for _ in range(steps):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            spin()
            e0.record()
            pfss.aes128_ctr(rk, 5, 7, blocks, bitsliced=bs, out=outs[name])
            e1.record()
            torch.cuda.synchronize()
            ms.append(e0.elapsed_time(e1))
        res[name + "_ms"] = float(np.median(ms))
        res[name + "_blocks_per_s"] = blocks / (res[name + "_ms"] / 1e3)
    res["bitsliced_over_ttable"] = res["bitsliced_ms"] / res["ttable_ms"]
    same = bool(torch.equal(outs["ttable"], outs["bitsliced"]))
    res["check"] = "ok" if same else "MISMATCH"
    return res


def main():
    a = parse()
    if a.gpus != 1:
        print("bench.py: measures one GPU only (got --gpus %d); sharding the key "
              "batch and the layer across GPUs is not implemented" % a.gpus)
        sys.exit(2)
    if a.calibrate_copy:
        calibrate_copy()
        return
    if a.only:
        import torch  # noqa: F401  (initialises the device before the library)

        from suf_amd import native

        native.call("sufhip_init", 0)
        cpu_s = 0.0 if a.no_cpu else a.cpu_seconds / 2
        sh = not a.no_shared
        run = {"spline": lambda: bench_spline(a.steps, a.warmup, cpu_seconds=cpu_s, shared=sh),
               "matmul": lambda: bench_matmul(a.steps, a.warmup, cpu_seconds=cpu_s),
               "softmax_ln": lambda: bench_softmax_ln(a.steps, a.warmup, cpu=not a.no_cpu,
                                                      shared=sh),
               "layer": lambda: bench_layer(a.steps, a.warmup, cpu=not a.no_cpu,
                                            shared=sh),
               "aes": lambda: bench_aes(a.steps, a.warmup)}[a.only]
        res = run()
        print(json.dumps({"only": a.only, **res}), flush=True)
        sys.exit(0 if res["check"] in ("ok", "not run (--no-cpu)") else 1)
    import numpy as np
    import torch

    from suf_amd import native, pfss

    native.call("sufhip_init", 0)
    n = a.n
    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    r_in = pfss.host_mt19937_64(1, n)
    x = pfss.host_normal_fixed(2, 1.0, 0.0, 12, n)
    xhat = (x + r_in).astype(np.uint64)
    seeds = pfss.host_mt19937_64(4, 4 * n).view(np.uint8).reshape(n, 32)

    def d(arr):
        arr = np.ascontiguousarray(arr)
        if arr.dtype == np.uint64:
            arr = arr.view(np.int64)
        return torch.from_numpy(arr.copy()).cuda()

    d_alpha, d_xhat, d_seeds = d(r_in), d(xhat), d(seeds)
    d_beta = d(np.array([1], dtype=np.uint8))
    kb = pfss.dcf_key_bytes(64, 1)

    # Keygen (dealer), once, on the device.
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    k0, k1 = pfss.dcf_gen(native.GROUP_XOR, 64, state, d_alpha, d_beta, d_seeds)
    e1.record()
    torch.cuda.synchronize()
    keygen_ms = e0.elapsed_time(e1)

    out0 = torch.empty(n, dtype=torch.uint8, device="cuda")
    out1 = torch.empty(n, dtype=torch.uint8, device="cuda")

    def step(evs=None):
        if evs is not None:
            evs[0].record()
        pfss.dcf_eval(native.GROUP_XOR, 64, 1, state, k0, d_xhat, native.DCF_OUT_BIT, out=out0)
        if evs is not None:
            evs[1].record()
        pfss.dcf_eval(native.GROUP_XOR, 64, 1, state, k1, d_xhat, native.DCF_OUT_BIT, out=out1)
        if evs is not None:
            evs[2].record()

    for _ in range(a.warmup):
        step()
    torch.cuda.synchronize()
    evs = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(a.steps)]
    t_start, t_stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record()
    for s in range(a.steps):
        step(evs[s])
    t_stop.record()
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_stop)
    launch_ms = [e[0].elapsed_time(e[1]) for e in evs] + [e[1].elapsed_time(e[2]) for e in evs]
    kern_ms = float(np.mean(launch_ms))

    # Reconstruct and check (outside the timed region).
    rec = (out0 ^ out1).cpu().numpy()
    ok = bool(np.array_equal(rec, (xhat < r_in).astype(np.uint8)))

    evals = 2 * n * a.steps
    value = evals / (total_ms / 1e3)
    key_bytes_per_launch = n * (kb + 8 + 1)
    achieved_gbps = key_bytes_per_launch / (kern_ms / 1e3) / 1e9
    line = {
        "metric": METRIC,
        "value": value,
        "unit": "evals/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": total_ms / a.steps,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": {
            "workload": "dcf_batch: N=2^20 myl7 DCF keys per party over Z_2^64, 2 parties",
            "N": n, "in_bits": 64, "lambda_bytes": 16, "group": "xor", "payload_bytes": 1,
            "key_bytes": kb, "out": "1 byte per eval (share byte 0 & 1)",
            "parallelism": "single GPU",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": achieved_gbps,
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": achieved_gbps / HBM_PEAK_GBPS,
            "traffic": MEASURED_TRAFFIC_BYTES if n == 1 << 20 else None,
            "kernel": "dcf_eval_bit_kernel",
            "kernel_ms": kern_ms,
            "bytes_per_launch": key_bytes_per_launch,
            "basis": "N x (2152 key + 8 xhat + 1 out) bytes",
            "note": "key bytes streamed per launch / launch time; the kernel is bound by "
                    "its LDS T-table reads and VALU AES work, see roofline_lds and roofline_valu",
        },
        # The pipes that bind the AES work: VALU lane-ops and LDS read bytes
        # per launch (counter totals for N = 2^20) over the measured launch time.
        "roofline_valu": {
            "bound": "valu",
            "achieved": DCF_VALU_INSTS * 64 / (kern_ms / 1e3) / 1e9 * (n / (1 << 20)),
            "peak": VALU_PEAK_GOPS,
            "unit": "Gop/s",
            "frac": DCF_VALU_INSTS * 64 / (kern_ms / 1e3) / 1e9 * (n / (1 << 20)) / VALU_PEAK_GOPS,
            "valu_insts_per_launch": DCF_VALU_INSTS,
            "aes_blocks_per_launch": n * 64 * 2,
        },
        "roofline_lds": {
            "bound": "lds",
            "achieved": DCF_LDS_INSTS * 256 / (kern_ms / 1e3) / 1e9 * (n / (1 << 20)),
            "peak": LDS_PEAK_GBPS,
            "unit": "GB/s",
            "frac": DCF_LDS_INSTS * 256 / (kern_ms / 1e3) / 1e9 * (n / (1 << 20)) / LDS_PEAK_GBPS,
            "lds_insts_per_launch": DCF_LDS_INSTS,
            "note": "256 bytes per wave64 4-byte LDS instruction; bank conflicts measured 0",
        },
        "keygen_ms": keygen_ms,
        "secure_layer_ms": None,
        "check": "ok" if ok else "MISMATCH",
    }
    progress("dcf batch: %.3g evals/s" % value)
    if not a.no_gates:
        gate_cpu = 0.0 if a.no_cpu else a.cpu_seconds / 2
        sh = not a.no_shared
        line["spline_gate"] = bench_spline(max(a.steps // 2, 1), 2, cpu_seconds=gate_cpu,
                                           shared=sh)
        progress("spline gate: %.4f ms" % line["spline_gate"]["ms"])
        line["beaver_matmul_trunc"] = bench_matmul(max(a.steps // 2, 1), 2, cpu_seconds=gate_cpu)
        progress("beaver matmul + trunc: %.4f ms" % line["beaver_matmul_trunc"]["ms"])
        line["softmax_layernorm"] = bench_softmax_ln(max(a.steps // 2, 1), 2, cpu=not a.no_cpu,
                                                     shared=sh)
        progress("softmax + layernorm: %.4f ms" % line["softmax_layernorm"]["ms"])
        line["secure_layer"] = bench_layer(max(a.steps // 2, 1), 2, cpu=not a.no_cpu, shared=sh)
        progress("secure layer: %.4f ms" % line["secure_layer"]["ms"])
        line["secure_layer_ms"] = line["secure_layer"]["ms"]
        line["secure_layer_note"] = ("one HIP-graph replay of suf_amd/layer.py's two-party "
                                     "layer (both parties, one GPU, each party's LUT "
                                     "keystreams its own); protocol deviations from "
                                     "transformer_layer_forward are listed in "
                                     "secure_layer.protocol_deviations")
        ok = ok and line["spline_gate"]["check"] in ("ok", "not run (--no-cpu)")
        ok = ok and line["beaver_matmul_trunc"]["check"] == "ok"
        ok = ok and line["softmax_layernorm"]["check"] in ("ok", "not run (--no-cpu)")
        ok = ok and line["secure_layer"]["check"] in ("ok", "not run (--no-cpu)")
    if not a.no_cpu:
        sample = 1 << 16
        g0 = out0[:sample].cpu().numpy()
        g1 = out1[:sample].cpu().numpy()
        line["cpu_baseline"] = cpu_baseline(k0[:sample].cpu().numpy(), k1[:sample].cpu().numpy(),
                                            xhat[:sample], g0, g1, a.cpu_seconds)
        refn = 1 << 12
        ref = cpu_baseline_reference(k0[:refn].cpu().numpy(), k1[:refn].cpu().numpy(),
                                     xhat[:refn], g0[:refn], g1[:refn], a.cpu_seconds / 2)
        if ref is not None:
            line["cpu_baseline_reference"] = ref
    print(json.dumps(line), flush=True)
    if not ok:
        sys.exit(1)


if __name__ == "__main__":
    main()
