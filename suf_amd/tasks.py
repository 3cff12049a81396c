"""Building blocks of SUF's task chains for two parties on one GPU.

The reference runs each gate as a PhaseTask per party over a local channel
(include/runtime/phase_tasks.hpp).  Here both parties live in one process on
one GPU, so every protocol round is one launch that does both parties' local
work and the open (libsuf_hip.so two-party kernels); these classes hold the
dealer material of one gate instance and issue those launches on torch's
current stream.

  Dealer       seeded std::mt19937_64 streams for one block's randomness
  Triples      Beaver triples, elementwise or row-broadcast
               (RowBroadcastTripleProvider, phase_tasks.hpp:1701-1712)
  Trunc        one truncation gate (TruncTask, phase_tasks.hpp:403-1166):
               both parties' keys, the key-only prepare and the finish
  CoeffLut     one coefficient interval LUT over a public masked input (the
               composite interval-LUT fast path, include/gates/composite_fss.hpp:
               1248-1384), rotated by the gate's r_in
  term/operand the generalised operands of sufhip_lin2 / sufhip_mul2x
"""
import numpy as np
import torch

from . import native, pfss

M64 = (1 << 64) - 1
LUT_TWEAK = 7  # seed_from_id tweak of interval LUT keys (cuda/pfss_backend_gpu.cu:508-515)


def stream_ptr():
    return torch.cuda.current_stream().cuda_stream


def ptr(t):
    return t.data_ptr() if t is not None else None


def dev(a, device="cuda"):
    """Host u64 / int64 numpy array -> device int64 tensor (same bits)."""
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int64).copy()).to(device)


def dev_i32(a, device="cuda"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32).copy()).to(device)


def split(v, s):
    """Additive split of v with party 0's share s."""
    return s & M64, (v - s) & M64


class Dealer:
    """Randomness of one block: draw k uses the first words of
    std::mt19937_64(seed * 0x9e3779b97f4a7c15 + k)."""

    def __init__(self, seed):
        self.seed = int(seed)
        self.k = 0

    def words(self, n):
        self.k += 1
        return pfss.host_mt19937_64((self.seed * 0x9E3779B97F4A7C15 + self.k) & M64, n)

    def word(self):
        return int(self.words(1)[0])


def term(pair, index=None, stride=1, off=0, shift=0, neg=False, length=None, mul=1):
    """sufhip_term2 over a pair of device tensors (party 0, party 1)."""
    t = native.Term2()
    if pair is None:
        return t
    t.p[0], t.p[1] = pair[0].data_ptr(), pair[1].data_ptr()
    t.index = index.data_ptr() if index is not None else None
    t.len = length if length is not None else pair[0].numel() // stride
    t.stride, t.off, t.shift, t.negate = stride, off, shift, 1 if neg else 0
    t.mul = mul & M64
    return t


def operand(*terms, const=0):
    """sufhip_operand2: up to two terms plus a public constant (party 0)."""
    if len(terms) > 2:
        raise ValueError("an operand holds at most two terms")
    o = native.Operand2()
    for k, t in enumerate(terms):
        o.t[k] = t
    o.party0_const = const & M64
    return o


def _open_target(into, xhat, mask):
    """into = (Trunc, out pair): the open feeds that truncation gate.
    Returns (epilogue struct or None, open buffer, mask, finish-afterwards)."""
    if into is None:
        return None, xhat, mask, None
    tr, y = into
    if tr.has_table():
        return tr.epilogue(y), None, tr.mask, None
    return None, tr.zhat_buf(), tr.mask, (tr, y)


def _after(fin):
    if fin is not None:
        tr, y = fin
        tr.finish(tr.zhat_buf(), y)


def lin2(x, n, out=None, xhat=None, mask=0, into=None):
    """Operand shares (out) and/or their masked open (xhat), or with
    into = (Trunc, y) the open truncated into y."""
    epi, hat, mask, fin = _open_target(into, xhat, mask)
    native.call("sufhip_lin2", native.ctypes.byref(x), n,
                ptr(out[0]) if out is not None else None,
                ptr(out[1]) if out is not None else None, ptr(hat), mask & M64,
                native.ctypes.byref(epi) if epi is not None else None, stream_ptr())
    _after(fin)


def kb_planes_out(spec):
    """sufhip_kb_planes from (planes, batches, rows, cols, k_is_col) or
    (planes, batches, rows, cols, k_is_col, planes_a0, a0): the latter also
    writes the planes of open + a0 (a0 a device tensor indexed like the
    open), or none."""
    o = native.KbPlanes()
    if spec is not None:
        o.planes = ptr(spec[0])
        o.batches, o.rows, o.cols, o.k_is_col = spec[1], spec[2], spec[3], int(spec[4])
        if len(spec) > 5:
            o.planes_a0, o.a0 = ptr(spec[5]), ptr(spec[6])
    return o


def lin2_batch(jobs):
    """Up to four independent lin2 opens in one launch: jobs of (operand, n,
    xhat, mask) or (operand, n, xhat, mask, planes): planes = (buffer,
    batches, rows, cols, k_is_col) also writes the open as a two-party
    product operand's digit planes (xhat may then be None)."""
    arr = (native.Lin2Job * len(jobs))()
    for k, jb in enumerate(jobs):
        x, n, xhat, mask = jb[:4]
        arr[k].x, arr[k].n, arr[k].xhat, arr[k].mask = x, n, ptr(xhat), mask & M64
        arr[k].xhat_planes = kb_planes_out(jb[4] if len(jb) > 4 else None)
    native.call("sufhip_lin2_batch", arr, len(jobs), stream_ptr())


def mul2x(u, v, tri, n, z=None, zhat=None, open_mask=0, z_add=None, into=None):
    """Beaver product of two operands with triple `tri` (a Triples); writes
    the shares to z (pair), the masked open of the product to zhat, or with
    into = (Trunc, y) the open truncated into y."""
    epi, hat, mask, fin = _open_target(into, zhat, open_mask)
    a = native.Mul2xArgs()
    a.u, a.v = u, v
    a.a, a.b, a.c = tri.terms()
    if z_add is not None:
        a.z_add = z_add
    if z is not None:
        a.z[0], a.z[1] = ptr(z[0]), ptr(z[1])
    a.zhat = ptr(hat)
    a.open_mask = mask & M64
    a.trunc = native.ctypes.cast(native.ctypes.pointer(epi), native.c_vp) if epi is not None \
        else None
    native.call("sufhip_mul2x", native.ctypes.byref(a), n, stream_ptr())
    _after(fin)


def row_sum2(x, rows, cols=0, offsets=None, mul_const=1, sums=None, hat=None, mask=0,
             into=None):
    epi, hat, mask, fin = _open_target(into, hat, mask)
    native.call("sufhip_row_sum2", native.ctypes.byref(x), rows, cols, ptr(offsets),
                mul_const & M64, ptr(sums[0]) if sums is not None else None,
                ptr(sums[1]) if sums is not None else None, ptr(hat), mask & M64,
                native.ctypes.byref(epi) if epi is not None else None, stream_ptr())
    _after(fin)


class Triples:
    """Beaver triples for n products.  a, c per element; b per element, or
    per row when row_of (host int array: the row of each element) is given,
    with c_i = a_i * b_row(i) (the row-broadcast triple).  Party 0 holds the
    drawn shares, party 1 the differences."""

    def __init__(self, dealer, n, row_of=None, device="cuda"):
        self.n = n
        nb = n if row_of is None else int(np.max(row_of)) + 1 if len(row_of) else 1
        a = dealer.words(n)
        b = dealer.words(nb)
        c = a * (b if row_of is None else b[np.asarray(row_of)])
        a0, b0, c0 = dealer.words(n), dealer.words(nb), dealer.words(n)
        self.a = (dev(a0, device), dev(a - a0, device))
        self.b = (dev(b0, device), dev(b - b0, device))
        self.c = (dev(c0, device), dev(c - c0, device))
        self.row_index = None if row_of is None else dev_i32(row_of, device)
        self.host = {"a": a, "b": b, "c": c, "a0": a0, "b0": b0, "c0": c0}

    def terms(self):
        return term(self.a), term(self.b, index=self.row_index), term(self.c)

    def shares(self, p):
        """Host copies of party p's (a, b, c) shares (tests)."""
        h = self.host
        if p == 0:
            return h["a0"], h["b0"], h["c0"]
        return ((h["a"] - h["a0"]).astype(np.uint64), (h["b"] - h["b0"]).astype(np.uint64),
                (h["c"] - h["c0"]).astype(np.uint64))


TABLE_BITS = 14  # carry keys this wide are prepared as full-domain tables


class Trunc:
    """One truncation gate (scalar mask r) over n elements, both parties."""

    def __init__(self, dealer, frac_bits, n, prg_state, kind=native.TRUNC_GAPARS,
                 device="cuda", rnd=None):
        self.kind, self.f, self.n = kind, frac_bits, n
        self.device = device
        self.prg_state = bytes(prg_state)
        self.rnd = np.ascontiguousarray(rnd, dtype=np.uint64) if rnd is not None else \
            dealer.words(native.TRUNC_RAND_WORDS)
        self.mask = int(self.rnd[0])  # r = r_0 + r_1: the open's mask
        self.keys = pfss.trunc_gen(kind, frac_bits, self.prg_state, self.rnd, device)
        self.work_bytes = native.load().sufhip_trunc_work_bytes(frac_bits, n)
        self.work = [torch.empty(max(2, (self.work_bytes + 15) // 8), dtype=torch.int64,
                                 device=device) for _ in range(2)]
        self._state = pfss._state_buf(self.prg_state)
        self._zhat = None

    def has_table(self):
        """The finish is one table read that other launches can fold in."""
        return self.kind == native.TRUNC_GAPARS and self.f <= TABLE_BITS

    def zhat_buf(self):
        if self._zhat is None:
            self._zhat = torch.empty(self.n, dtype=torch.int64, device=self.device)
        return self._zhat

    def jobs(self):
        """sufhip_trunc_job of both parties' keys (key-only half)."""
        out = []
        for p in (0, 1):
            j = native.TruncJob()
            j.kind, j.frac_bits = self.kind, self.f
            j.d_key, j.key_bytes = ptr(self.keys[p]), self.keys[p].numel()
            j.n, j.d_work, j.work_bytes = self.n, ptr(self.work[p]), self.work_bytes
            out.append(j)
        return out

    def epilogue(self, y, add=None):
        """The sufhip_trunc_epilogue writing the gate's outputs to the pair y
        (plus the pair `add`, if given)."""
        e = native.TruncEpilogue()
        e.key[0], e.key[1] = ptr(self.keys[0]), ptr(self.keys[1])
        e.table[0], e.table[1] = ptr(self.work[0]), ptr(self.work[1])
        e.work_bytes = self.work_bytes
        e.frac_bits = self.f
        e.y[0], e.y[1] = ptr(y[0]), ptr(y[1])
        if add is not None:
            e.add[0], e.add[1] = ptr(add[0]), ptr(add[1])
        return e

    def prepare(self, stream=None):
        """Key-only half (both parties) on `stream` (default: current)."""
        prepare_batch([self], stream)

    def finish(self, xhat, out):
        """Both parties' outputs at the masked open xhat (one launch)."""
        native.call("sufhip_trunc_finish2", self.kind, self.f, self._state, ptr(self.keys[0]),
                    ptr(self.keys[1]), self.keys[0].numel(), ptr(xhat), self.n, ptr(out[0]),
                    ptr(out[1]), ptr(self.work[0]), ptr(self.work[1]), self.work_bytes,
                    stream_ptr())


def trunc_jobs(truncs):
    """(PRG state buffer, sufhip_trunc_job array, count) of the key-only
    halves of truncation gates that share one PRG state."""
    state = truncs[0].prg_state
    if any(t.prg_state != state for t in truncs):
        raise ValueError("prepare_batch: gates with different PRG states")
    jobs = [j for t in truncs for j in t.jobs()]
    return truncs[0]._state, (native.TruncJob * len(jobs))(*jobs), len(jobs)


def prepare_batch(truncs, stream=None):
    """The key-only halves of many truncation gates (same PRG state) in one
    batched launch sequence on `stream` (default: current)."""
    if not truncs:
        return
    state, arr, count = trunc_jobs(truncs)
    s = stream.cuda_stream if stream is not None else stream_ptr()
    native.call("sufhip_trunc_prepare_batch", state, arr, count, s)


class Prepared:
    """Key-only halves of a block's truncation gates issued on a side stream
    (in batches, in order of need); wait(k) makes the current stream wait for
    batch k.  With upfront = u, only the first u batches are issued now and
    release() issues the rest once the current stream's work so far is done
    (so that they overlap later work instead of the next kernels).  With
    side = None the batches are issued on the current stream itself and
    wait() has nothing to order."""

    def __init__(self, side, batches, upfront=None):
        self.side = side
        self.batches = list(batches)
        self.events = [None] * len(self.batches)
        self.issued = 0
        self._issue(len(self.batches) if upfront is None else upfront)

    def _issue(self, upto):
        if self.side is None:
            for k in range(self.issued, upto):
                prepare_batch(self.batches[k])
            self.issued = max(self.issued, upto)
            return
        start = torch.cuda.Event()
        start.record()
        self.side.wait_event(start)
        for k in range(self.issued, upto):
            prepare_batch(self.batches[k], self.side)
            ev = torch.cuda.Event()
            ev.record(self.side)
            self.events[k] = ev
        self.issued = max(self.issued, upto)

    def release(self):
        self._issue(len(self.batches))

    def wait(self, k=0):
        if k >= self.issued:
            raise RuntimeError("Prepared.wait: batch %d was not released" % k)
        if self.side is not None:
            torch.cuda.current_stream().wait_event(self.events[k])


def rotated_lut(alpha, coeffs, r_in):
    """Interval LUT geometry over x^ = x + r_in for pieces [alpha_i,
    alpha_{i+1}) (the last to 2^64) with coefficient rows `coeffs`: cutpoints
    [k + 1] (the last is the 2^64 sentinel 0) and payload [k][words]
    (rotation and wrap split as src/compiler/suf_to_pfss.cpp:506-523)."""
    ivs = []
    bounds = [int(a) for a in alpha] + [1 << 64]
    for i in range(len(alpha)):
        s = (bounds[i] + r_in) & M64
        e = (bounds[i + 1] + r_in) & M64
        pay = [int(v) & M64 for v in coeffs[i]]
        if s < e:
            ivs.append((s, e, pay))
        else:
            ivs.append((s, 0, pay))
            if e != 0:
                ivs.append((0, e, pay))
    ivs.sort(key=lambda t: t[0])
    cuts = [ivs[0][0]] + [hi for _, hi, _ in ivs]
    payload = [w for _, _, pay in ivs for w in pay]
    return np.array(cuts, dtype=np.uint64), np.array(payload, dtype=np.uint64), len(ivs)


class CoeffLut:
    """Both parties' broadcast interval-LUT keys returning the coefficient
    row of x's piece at the public x^ = x + r_in.  mask = r_in."""

    def __init__(self, dealer, alpha, coeffs, device="cuda", coeffs_for_rin=None):
        self.words = int(np.asarray(coeffs).shape[1])
        r_in = dealer.word()
        self.mask = r_in
        rows = coeffs_for_rin(r_in) if coeffs_for_rin is not None else coeffs
        cuts, payload, k = rotated_lut(alpha, rows, r_in)
        self.intervals = k
        lib = native.load()
        self.key_bytes = lib.sufhip_interval_lut_key_bytes(k, self.words)
        self.nonce = dealer.word()
        seed16 = native.ctypes.create_string_buffer(16)
        lib.sufhip_seed_from_id(self.nonce, LUT_TWEAK, seed16)
        self.blobs = []
        self.keys = []
        for party in (0, 1):
            blob = np.zeros(self.key_bytes, dtype=np.uint8)
            native.call("sufhip_interval_lut_build_key", party, self.nonce, 64, self.words,
                        cuts.ctypes.data, k, payload.ctypes.data, seed16, blob.ctypes.data)
            self.blobs.append(blob)
            self.keys.append(torch.from_numpy(blob.view(np.int64).copy()).to(device)
                             .view(torch.uint8))

    def eval2(self, xhat, n, out, x=None):
        """Both parties' rows at the masked open: xhat (device tensor), or
        with x (an operand) at x_0 + x_1 + mask computed in the same launch.
        out: pair of int64 [n * words] tensors (AoS rows)."""
        native.call("sufhip_interval_lut_eval2", ptr(self.keys[0]), ptr(self.keys[1]),
                    self.key_bytes, self.intervals, self.words,
                    native.ctypes.byref(x) if x is not None else None, ptr(xhat),
                    self.mask & M64, n, ptr(out[0]), ptr(out[1]), stream_ptr())


def relu_coeffs_for(r_in):
    """ReLU (make_relu_value_suf_u64, include/gates/relu_gate.hpp:9-44) as
    public-x^ coefficients: x = x^ - r_in on [0, 2^63) -> (-r_in, 1), 0 on
    [2^63, 2^64) -> (0, 0) (shift_coeffs_to_public_hatx,
    src/compiler/suf_to_pfss.cpp:193-243)."""
    return [[(-r_in) & M64, 1], [0, 0]]


RELU_ALPHA = np.array([0, 1 << 63], dtype=np.uint64)


def pair(n, device="cuda", width=1):
    return tuple(torch.empty(n * width, dtype=torch.int64, device=device) for _ in range(2))


def capture(fn, warmup=1):
    """Records fn() (launches on torch's current stream, side streams joined
    by events) into a HIP graph; replay() then reissues the whole chain with
    one launch.  fn must allocate nothing and clear no memory with memset
    (every entry point of libsuf_hip.so qualifies).  Runs fn `warmup` times
    eagerly first."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(warmup):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g


class AosTriples:
    """Elementwise triples stored as {a, b, c} per element (the AoS layout of
    launch_beaver_mul_aos_kernel, include/runtime/cuda_primitives.hpp:29-35):
    pair of int64 [n * 3] tensors."""

    def __init__(self, pair_aos):
        self.t = pair_aos

    def terms(self):
        return (term(self.t, stride=3, off=0), term(self.t, stride=3, off=1),
                term(self.t, stride=3, off=2))


def x_planes(planes=None):
    """sufhip_x_planes from (buffer, cols), or none."""
    xp = native.XPlanes()
    if planes is not None:
        xp.planes, xp.cols = ptr(planes[0]), planes[1]
    return xp


def chain2(kind, f, x, n, lut_keys, lut_key_bytes, intervals, lut_mask, triples, truncs, out,
           planes=None, write_out=True):
    """A whole elementwise gate chain (sufhip_gate_chain2) for both parties:
    kind native.CHAIN_*, x the input operand, lut_keys both parties' LUT
    blobs, triples / truncs the chain's products and truncation gates in
    order, out the output pair; planes = (buffer, cols): the output also as a
    public-weight product's digit planes (write_out False: only those)."""
    a = chain2_args(kind, f, x, n, lut_keys, lut_key_bytes, intervals, lut_mask, triples, truncs,
                    out)
    a.out_planes = x_planes(planes)
    if not write_out:
        a.out[0] = a.out[1] = None
    native.call("sufhip_gate_chain2", native.ctypes.byref(a), stream_ptr())


def triple2(tri):
    """sufhip_triple2 of a Triples (b per row when it is row-broadcast)."""
    t = native.Triple2()
    for p in (0, 1):
        t.a[p], t.b[p], t.c[p] = ptr(tri.a[p]), ptr(tri.b[p]), ptr(tri.c[p])
    return t


def chain2_args(kind, f, x, n, lut_keys, lut_key_bytes, intervals, lut_mask, triples, truncs,
                out):
    """The sufhip_chain2_args of chain2 (x None: an empty operand, for a
    chain embedded in a block launch)."""
    a = native.Chain2Args()
    a.kind, a.frac_bits, a.n = kind, f, n
    if x is not None:
        a.x = x
    a.lut[0], a.lut[1] = ptr(lut_keys[0]), ptr(lut_keys[1])
    a.lut_key_bytes, a.intervals, a.lut_mask = lut_key_bytes, intervals, lut_mask & M64
    for k, t in enumerate(triples):
        a.a[k], a.b[k], a.c[k] = t.terms()
    for k, tr in enumerate(truncs):
        a.trunc[k] = tr.epilogue(out)
        a.trunc_mask[k] = tr.mask & M64
    a.out[0], a.out[1] = ptr(out[0]), ptr(out[1])
    return a
