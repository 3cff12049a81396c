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
MEASURED_TRAFFIC_BYTES = 1256045.2 * 1024 * 2.0 + 1233.0 * 1024 * 1.0
# Instructions per dcf_eval_bit_kernel launch at N = 2^20 (rocprofv3 --pmc
# SQ_INSTS_VALU SQ_INSTS_LDS, same profile file): fixed by the compiled kernel
# and N, so lane-ops per second follow from the measured launch time.
DCF_VALU_INSTS = 534897920
DCF_LDS_INSTS = 330368256
VALU_PEAK_GOPS = 256 * 64 * 2.4  # 256 CUs x 4 SIMDs x 16 lanes x 2.4 GHz, 32-bit integer ops
# LDS: 128 bytes per clock per CU (a wave64 4-byte read every 2 clocks, as
# measured for this kernel's random-index reads) x 256 CUs x 2.4 GHz.
LDS_PEAK_GBPS = 256 * 128 * 2.4


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
    ap.add_argument("--only", choices=["spline", "matmul", "softmax_ln", "layer"],
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


def bench_spline(steps, warmup, n=1 << 20, frac_bits=12, cpu_seconds=0.0):
    """The spline gate (interval LUT + three Beaver products + GapARS by f and
    2f) for both parties on N = 2^20 inputs x = clip(3 N(0,1), +-8) in Q12
    (Box-Muller on mt(5)); coefficients from mt(6); dealer randomness mt(7).
    Returns ms per gate evaluation (both parties) and the reconstruction check."""
    import numpy as np
    import torch

    from suf_amd import pfss, spline

    state = bytes((pfss.host_mt19937_64(3, 128) & np.uint64(0xFF)).astype(np.uint8))
    alpha, coeffs = spline.spline_spec(frac_bits, seed=6)
    x = pfss.host_normal_fixed(5, 3.0, 8.0, frac_bits, n)
    x0 = pfss.host_mt19937_64(8, n)
    x1 = (x - x0).astype(np.uint64)
    from suf_amd import tasks

    gate = spline.SplineGate(n, alpha, coeffs, state, frac_bits, seed=7)
    xd = [torch.from_numpy(v.view(np.int64).copy()).cuda() for v in (x0, x1)]
    out = [torch.empty(n, dtype=torch.int64, device="cuda") for _ in range(2)]

    def run():
        # The truncations' key-only halves first, on the same stream.
        gate.eval2(xd, out, prep=(tasks.Prepared(None, [gate.truncs()]), 0))

    ms, eager_ms = _graph_ms(run, steps, warmup)
    rec = (out[0].cpu().numpy().view(np.uint64) + out[1].cpu().numpy().view(np.uint64))
    ok = bool(np.array_equal(rec.astype(np.uint64),
                             spline.spline_eval_ref(alpha, coeffs, x, frac_bits)))
    res = {"ms": ms, "eager_ms": eager_ms, "n": n, "frac_bits": frac_bits,
           "intervals": int(gate.intervals),
           "trunc": "GapARS f=%d (x3: the 2f truncation as two f truncations)" % frac_bits,
           "steps": steps, "check": "ok" if ok else "MISMATCH"}
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_spline_baseline(gate, state, x0, x1,
                                                  [out[0].cpu().numpy(), out[1].cpu().numpy()],
                                                  cpu_seconds)
    return res


def cpu_spline_baseline(gate, state, x0, x1, gpu_out, seconds):
    """The same two-party spline gate on the host with the oracle's plain-C
    restatement of each step (interval LUT, Beaver products, truncation gate
    with its DCF walks), one thread, on consecutive 1024-element chunks of the
    batch until the time budget is used; shares compared with the GPU's."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    prg = ol.Prg(state)
    f = gate.f
    lut = [gate.lut[p].cpu().numpy() for p in (0, 1)]
    tri = [[t.cpu().numpy().view(np.uint64).reshape(-1, 3) for t in pair] for pair in gate.triples]
    tk = [[k.cpu().numpy() for k in t.keys] for t in gate.trunc]
    rin = sum(gate.rin) & ((1 << 64) - 1)
    t_rin = [t.mask for t in gate.trunc]
    sh = np.uint64(f)
    chunk, done, mism = 1024, 0, 0
    t0 = time.perf_counter()
    while done + chunk <= x0.size:
        sl = slice(done, done + chunk)
        a0, a1 = x0[sl], x1[sl]
        xhat = (a0 + a1 + np.uint64(rin)).astype(np.uint64)
        C = [ol.lut_eval(lut[p], gate.lut_key_bytes, 1, xhat, 4, idx0=done).reshape(chunk, 4)
             for p in (0, 1)]

        def mul(u, v, t):
            t = [t[0][sl], t[1][sl]]
            d = (u[0] - t[0][:, 0]) + (u[1] - t[1][:, 0])
            e = (v[0] - t[0][:, 1]) + (v[1] - t[1][:, 1])
            return [ol.beaver_mul(p, t[p][:, 0], t[p][:, 1], t[p][:, 2], d, e) for p in (0, 1)]

        u = mul([C[0][:, 3], C[1][:, 3]], [a0, a1], tri[0])
        u = [u[p] + (C[p][:, 2] << sh) for p in (0, 1)]
        pz = mul(u, [a0, a1], tri[1])
        phat = (pz[0] + pz[1] + np.uint64(t_rin[0])).astype(np.uint64)
        y = [ol.trunc_eval(prg, ol.TRUNC_GAPARS, f, tk[0][p], phat) for p in (0, 1)]
        q = [y[p] + (C[p][:, 1] << sh) for p in (0, 1)]
        rz = mul(q, [a0, a1], tri[2])
        rhat = (rz[0] + rz[1] + np.uint64(t_rin[1])).astype(np.uint64)
        y2 = [ol.trunc_eval(prg, ol.TRUNC_GAPARS, f, tk[1][p], rhat) for p in (0, 1)]
        z3 = [(y2[p] + (C[p][:, 0] << sh)).astype(np.uint64) for p in (0, 1)]
        zhat = (z3[0] + z3[1] + np.uint64(t_rin[2])).astype(np.uint64)
        for p in (0, 1):
            y3 = ol.trunc_eval(prg, ol.TRUNC_GAPARS, f, tk[2][p], zhat)
            mism += int(np.count_nonzero(y3 != gpu_out[p][sl].view(np.uint64)))
        done += chunk
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {"value": done / dt, "unit": "gate elements/s (both parties)", "cores": 1,
            "kind": "port", "ms_per_2p20": (1 << 20) / (done / dt) * 1e3,
            "sample": "%d of the 2^20 elements (oracle C restatement of LUT, Beaver and "
                      "truncation-gate steps, one thread); shares compared with the GPU: "
                      "%d mismatches" % (done, mism), "mismatches": mism}


def bench_matmul(steps, warmup, M=128, K=768, N=3072, frac_bits=12, cpu_seconds=0.0):
    """Beaver matmul + GapARS truncation for both parties: X [128 x 768] =
    round(N(0,1) 2^12) (mt(8)), W [768 x 3072] = round(N(0,0.02) 2^12) (mt(9)),
    both additively shared (mt(108), mt(109)); triples and truncation key from
    mt(10), mt(11).  Returns ms per evaluation and the reconstruction check."""
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
    # The product's own time (eager, events around it), then the whole gate
    # as one graph replay.
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    for s in range(steps):
        g.eval2(Xd, Wd, out, events=ev[s])
    torch.cuda.synchronize()
    mm_ms = float(np.mean([a.elapsed_time(b) for a, b in ev]))
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
    if cpu_seconds > 0:
        res["cpu_baseline"] = cpu_matmul_baseline(g, state, Xd, Wd, out, cpu_seconds)
    return res


def cpu_matmul_baseline(g, state, Xd, Wd, out, seconds):
    """Beaver matmul + truncation on the host: the oracle's OpenMP u64 matmul
    (src/nn/matmul_beaver.cpp:139-161 semantics) for both parties and the
    oracle truncation gate, on the first rows of the product (8 rows at a
    time) until the time budget is used; outputs compared with the GPU's."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    threads = min(os.cpu_count() or 1, 16)
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
    rows, mism = 0, 0
    t0 = time.perf_counter()
    while rows + 8 <= M:
        r = slice(rows, rows + 8)
        D = ((X[0][r] - A[0][r]) + (X[1][r] - A[1][r])).astype(np.uint64)
        Z = [ol.beaver_matmul(p, D, E, A[p][r], B[p], C[p][r], 1, 8, K, N, threads=threads)
             for p in (0, 1)]
        zhat = (Z[0] + Z[1] + np.uint64(rin)).astype(np.uint64)
        for p in (0, 1):
            y = ol.trunc_eval(prg, ol.TRUNC_GAPARS, f, keys[p], zhat)
            mism += int(np.count_nonzero(y != gpu[p][r].ravel()))
        rows += 8
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    macs = 2 * 2 * rows * K * N
    return {"value": macs / dt, "unit": "u64 MAC/s (both parties, with truncation)",
            "cores": threads, "kind": "port", "ms_full_shape": dt * M / rows * 1e3,
            "sample": "%d of the %d output rows (oracle C matmul, OpenMP %d threads, then the "
                      "oracle truncation gate); outputs compared with the GPU: %d mismatches"
                      % (rows, M, threads, mism), "mismatches": mism}


def bench_softmax_ln(steps, warmup, frac_bits=12, cpu=True):
    """Softmax over 12 heads x 128 x 128 causal score rows (scores
    round(N(0,2) 2^12), mt(11)) followed by LayerNorm over 128 x 768
    (round(N(0,1) 2^12), mt(12)), both parties; shares from mt(111), mt(121);
    dealer material from suf_amd.tasks.Dealer(11), Dealer(12).  Returns ms
    per block (softmax + LayerNorm) and each part."""
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
            ev[0].record()
        sm.eval2(sin, sout, prep=prep)
        if ev:
            ev[1].record()
        ln.eval2(lin, lout, prep=prep)
        if ev:
            ev[2].record()

    ms, eager_ms = _graph_ms(run, steps, warmup)
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(steps)]
    for s in range(steps):
        run(ev[s])
    torch.cuda.synchronize()
    sm_ms = float(np.mean([e[0].elapsed_time(e[1]) for e in ev]))
    ln_ms = float(np.mean([e[1].elapsed_time(e[2]) for e in ev]))
    res = {"ms": ms, "eager_ms": eager_ms, "softmax_ms": sm_ms, "layernorm_ms": ln_ms,
           "split": "softmax_ms / layernorm_ms: eager, without the shared prepare walk",
           "softmax_shape": "12 heads x 128 causal rows (%d scores)" % n_sm,
           "layernorm_shape": [rows, cols], "frac_bits": frac_bits, "steps": steps,
           "check": "not run (--no-cpu)"}
    if cpu:
        res.update(cpu_softmax_ln_baseline(state, sm, ln, (s0, s1), (l0, l1), sc, xl, sout, lout,
                                           frac_bits))
    return res


def cpu_softmax_ln_baseline(state, sm, ln, sx, lx, sc, xl, sout, lout, f):
    """The same two-party softmax and LayerNorm chains on the host, composed
    from the oracle's plain-C steps (interval LUT, Beaver, truncation gate with
    its DCF walks), one thread, over the whole batch; shares compared with the
    GPU's, and the reconstruction checked against the fixed-point closed form."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import fixed_point as fp
    import oracle_lib as ol
    import twoparty_oracle as tp

    h = lambda t: t.cpu().numpy().view(np.uint64)
    t0 = time.perf_counter()
    prob, _ = tp.softmax2(ol.Prg(state), sm, list(sx))
    t1 = time.perf_counter()
    y = tp.layernorm2(ol.Prg(state), ln, list(lx))
    t2 = time.perf_counter()
    mism = sum(int(np.count_nonzero(prob[p] != h(sout[p]))) for p in (0, 1))
    mism += sum(int(np.count_nonzero(y[p] != h(lout[p]))) for p in (0, 1))
    want_p, _ = fp.softmax_block(sc, sm.offsets, sm.nexp_table, sm.recip.table, f)
    want_y, _ = fp.layernorm(xl, ln.rows, ln.cols, f, ln.inv_len, ln.eps_q, ln.rsqrt.table)
    rec_ok = (np.array_equal((h(sout[0]) + h(sout[1])).astype(np.uint64), want_p.view(np.uint64))
              and np.array_equal((h(lout[0]) + h(lout[1])).astype(np.uint64),
                                 want_y.view(np.uint64)))
    return {"check": "ok" if rec_ok and mism == 0 else "MISMATCH",
            "cpu_baseline": {"value": (t2 - t0) * 1e3, "unit": "ms per block (both parties)",
                             "softmax_ms": (t1 - t0) * 1e3, "layernorm_ms": (t2 - t1) * 1e3,
                             "cores": 1, "kind": "port",
                             "sample": "the whole block (oracle C restatement of the LUT, "
                                       "Beaver and truncation-gate steps, one thread); shares "
                                       "compared with the GPU: %d mismatches" % mism,
                             "mismatches": mism}}


def bench_layer(steps, warmup, frac_bits=12, cpu=True):
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
    dev = lambda v: torch.from_numpy(np.ascontiguousarray(v).view(np.int64).copy()).cuda()
    xin = (dev(x0), dev((x - x0).astype(np.uint64)))
    ly = layer.TransformerLayer(state, W, seq, d, heads, ffn, frac_bits, seed=13)
    out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    for _ in range(warmup):
        ly.eval2(xin, out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        ly.eval2(xin, out)
    e1.record()
    torch.cuda.synchronize()
    eager_ms = e0.elapsed_time(e1) / steps
    # Per-stage split of one more eager run (events between stages; launch
    # overhead included, so the stages sum to more than the graph replay).
    stages = ["ln1", "qkv", "attention", "out_proj+residual", "ln2", "w1", "gelu",
              "w2+residual"]
    m = []
    ly.eval2(xin, out, marks=m)
    torch.cuda.synchronize()
    per_stage = {stages[i]: m[i].elapsed_time(m[i + 1]) for i in range(len(stages))}
    eager_out = [out[0].cpu().numpy().copy(), out[1].cpu().numpy().copy()]
    g = tasks.capture(lambda: ly.eval2(xin, out))
    torch.cuda.synchronize()
    replay_ok = True
    for _ in range(2):  # replays agree with the eager result
        g.replay()
        torch.cuda.synchronize()
        replay_ok = replay_ok and all(np.array_equal(out[p].cpu().numpy(), eager_out[p])
                                      for p in (0, 1))
    e0.record()
    for _ in range(steps):
        g.replay()
    e1.record()
    torch.cuda.synchronize()
    graph_ms = e0.elapsed_time(e1) / steps
    res = {"ms": graph_ms, "eager_ms": eager_ms, "stages_eager_ms": per_stage,
           "shape": {"seq": seq, "hidden": d, "heads": heads, "ffn": ffn}, "frac_bits": frac_bits,
           "ring": "Z_2^64", "steps": steps, "graph_replays_match_eager": replay_ok,
           "check": "not run (--no-cpu)" if replay_ok else "MISMATCH"}
    if cpu:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import fixed_point as fp
        from suf_amd import tables

        tabs = {"nexp": tables.nexp_table(frac_bits), "recip": tables.recip_table(frac_bits),
                "rsqrt": tables.rsqrt_table(frac_bits), "gelu": tables.gelu_table(frac_bits)}
        t0 = time.perf_counter()
        want, _ = fp.transformer_layer(x, W, seq, d, heads, ffn, frac_bits, tabs,
                                       tables.inv_len_qf(d), tables.eps_qf())
        dt = time.perf_counter() - t0
        rec = (eager_out[0].view(np.uint64) + eager_out[1].view(np.uint64)).astype(np.uint64)
        ok = replay_ok and bool(np.array_equal(rec, want.view(np.uint64)))
        res["check"] = "ok" if ok else "MISMATCH"
        res["closed_form_cpu_ms"] = dt * 1e3
    return res


def cpu_baseline(keys0, keys1, xhat, gpu_bits0, gpu_bits1, seconds):
    """The reference's own myl7 batch evaluation (oracle/_ref, built from the
    reference sources), single thread as in Myl7FssBackend::eval_dcf_many_u64
    (include/proto/myl7_fss_backend.hpp:73-100), on a bounded sample."""
    import numpy as np

    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle_lib as ol

    state = ol.mt64_bytes(3, 128)
    chunk = 1024
    kb = keys0.shape[1]
    if ol.ref_available():
        ref = ol.ref_lib(ol.GROUP_XOR)
        ref.ref_prg_init(ol.ptr(state), 128)
        kind = "reference"

        def run(keys, xs, out):
            return ref.ref_adapter_eval_many(64, kb, ol.ptr(keys), ol.ptr(xs, ol.u64p), len(xs),
                                             1, ol.ptr(out))
    else:
        prg = ol.Prg(state.tobytes())
        kind = "port"

        def run(keys, xs, out):
            out[:] = ol.myl7_eval_many_bit(prg, 0, 64, keys, xs)
            return 0

    done = 0
    mismatches = 0
    t0 = time.perf_counter()
    i = 0
    n = keys0.shape[0]
    while True:
        lo = (i * chunk) % n
        hi = lo + chunk
        for keys, gb in ((keys0, gpu_bits0), (keys1, gpu_bits1)):
            out = np.zeros(chunk, dtype=np.uint8)
            k = np.ascontiguousarray(keys[lo:hi])
            x = np.ascontiguousarray(xhat[lo:hi])
            assert run(k, x, out) == 0
            mismatches += int(np.count_nonzero(out != gb[lo:hi]))
            done += chunk
        i += 1
        if time.perf_counter() - t0 >= seconds:
            break
    dt = time.perf_counter() - t0
    return {
        "value": done / dt,
        "unit": "evals/s",
        "cores": 1,
        "kind": kind,
        "sample": "%d DCF evals over the first %d keys per party of the same N=2^20 "
                  "batch (cycled), serial myl7 dcf_eval via OpenSSL EVP AES as the "
                  "reference batch loop does; shares compared with the GPU: %d mismatches"
                  % (done, n, mismatches),
        "mismatches": mismatches,
    }


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
        run = {"spline": lambda: bench_spline(a.steps, a.warmup, cpu_seconds=cpu_s),
               "matmul": lambda: bench_matmul(a.steps, a.warmup, cpu_seconds=cpu_s),
               "softmax_ln": lambda: bench_softmax_ln(a.steps, a.warmup, cpu=not a.no_cpu),
               "layer": lambda: bench_layer(a.steps, a.warmup, cpu=not a.no_cpu)}[a.only]
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
    if not a.no_gates:
        gate_cpu = 0.0 if a.no_cpu else a.cpu_seconds / 2
        line["spline_gate"] = bench_spline(max(a.steps // 2, 1), 2, cpu_seconds=gate_cpu)
        line["beaver_matmul_trunc"] = bench_matmul(max(a.steps // 2, 1), 2, cpu_seconds=gate_cpu)
        line["softmax_layernorm"] = bench_softmax_ln(max(a.steps // 2, 1), 2, cpu=not a.no_cpu)
        line["secure_layer"] = bench_layer(max(a.steps // 2, 1), 2, cpu=not a.no_cpu)
        line["secure_layer_ms"] = line["secure_layer"]["ms"]
        ok = ok and line["spline_gate"]["check"] == "ok"
        ok = ok and line["beaver_matmul_trunc"]["check"] == "ok"
        ok = ok and line["softmax_layernorm"]["check"] in ("ok", "not run (--no-cpu)")
        ok = ok and line["secure_layer"]["check"] in ("ok", "not run (--no-cpu)")
    if not a.no_cpu:
        sample = 1 << 14
        g0 = out0[:sample].cpu().numpy()
        g1 = out1[:sample].cpu().numpy()
        line["cpu_baseline"] = cpu_baseline(k0[:sample].cpu().numpy(), k1[:sample].cpu().numpy(),
                                            xhat[:sample], g0, g1, a.cpu_seconds)
    print(json.dumps(line), flush=True)
    if not ok:
        sys.exit(1)


if __name__ == "__main__":
    main()
