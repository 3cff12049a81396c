"""GPT-2-shaped secure transformer layer for two parties on one GPU, and its
new building blocks.

  * public-weight GEMM (int8 digit MFMA): each party's share equals
    X_p W mod 2^64 (numpy uint64 matmul wraps mod 2^64), the masked open
    equals their sum plus the mask, over 1-3 weight digits and sliced /
    unsliced grids;
  * two-party batched Beaver matmul: each party's share equals the oracle's
    beaver_matmul (orc_beaver_matmul) per batch, and reconstructs to X W;
  * attention core and the whole layer: reconstruction equals the closed
    form of oracle/fixed_point.py (small shapes and the config shape
    128 x 768, 12 heads, FFN 3072).
"""
import os
import sys

import numpy as np
import pytest
import torch

import oracle_lib as ol
from gpu_util import dev, say, u64
from suf_amd import layer, native, pfss, tables
from suf_amd.tasks import Dealer

sys.path.insert(0, os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                "oracle"))
import fixed_point as fp  # noqa: E402

pytestmark = pytest.mark.gpu

STATE = ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes()
F = 12


@pytest.fixture(scope="module", autouse=True)
def _init():
    native.call("sufhip_init", 0)


def _tabs():
    return {"nexp": tables.nexp_table(F), "recip": tables.recip_table(F),
            "rsqrt": tables.rsqrt_table(F), "gelu": tables.gelu_table(F)}


def _pair(x, seed):
    x = np.asarray(x).astype(np.uint64)
    x0 = pfss.host_mt19937_64(seed, x.size)
    return x0, (x - x0).astype(np.uint64)


@pytest.mark.parametrize("M,K,N,wmax", [(32, 64, 96, 100), (64, 96, 64, 30000),
                                        (128, 768, 2304, 400), (32, 32, 32, 1 << 20),
                                        (128, 3072, 768, 500),
                                        # N % 64 == 0 (LDS-shared form) with 1, 3, 4 weight digits
                                        (96, 64, 64, 1), (64, 128, 128, 1 << 20),
                                        (32, 224, 192, 1 << 30), (32, 1024, 64, 1 << 20)])
def test_public_matmul_shares(M, K, N, wmax):
    rng = np.random.default_rng(M + K + N)
    W = rng.integers(-wmax, wmax + 1, size=(K, N)).astype(np.int64)
    W[0, 0], W[-1, -1] = wmax, -wmax
    X0 = pfss.host_mt19937_64(M * 7 + 1, M * K).reshape(M, K)
    X1 = pfss.host_mt19937_64(M * 7 + 2, M * K).reshape(M, K)
    say("public matmul %dx%dx%d wmax=%d" % (M, K, N, wmax))
    pm = layer.PublicMatmulTrunc(M, K, N, W, Dealer(3), STATE, F)
    out = tuple(torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    zhat = torch.empty(M * N, dtype=torch.int64, device="cuda")
    mask = 0x1234567890ABCDEF
    xd = (dev(X0), dev(X1))
    pm.product2(xd, out=out)
    pm.product2(xd, zhat=zhat, mask=mask)
    Wu = W.view(np.uint64)
    want = [np.matmul(X0, Wu).ravel(), np.matmul(X1, Wu).ravel()]
    assert np.array_equal(u64(out[0]), want[0]) and np.array_equal(u64(out[1]), want[1])
    assert np.array_equal(u64(zhat), (want[0] + want[1] + np.uint64(mask)).astype(np.uint64))


def test_public_matmul_trunc_reconstructs():
    M, K, N = 64, 128, 96
    X = pfss.host_normal_fixed(71, 1.0, 0.0, F, M * K)
    W = pfss.host_normal_fixed(72, 0.05, 0.0, F, K * N).view(np.int64).reshape(K, N)
    x0, x1 = _pair(X, 73)
    say("public matmul + trunc %dx%dx%d" % (M, K, N))
    pm = layer.PublicMatmulTrunc(M, K, N, W, Dealer(4), STATE, F)
    pm.tr.prepare()
    out = tuple(torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    pm.eval2((dev(x0), dev(x1)), out)
    rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
    want = fp.matmul_shift(X.view(np.int64).reshape(M, K), W, F).ravel().view(np.uint64)
    assert np.array_equal(rec, want)
    # With a residual folded into the truncation's write: the same shares plus
    # the addend, per party.
    r = pfss.host_mt19937_64(74, 2 * M * N).reshape(2, M * N)
    res = (dev(r[0]), dev(r[1]))
    out2 = tuple(torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    pm.eval2((dev(x0), dev(x1)), out2, add=res)
    for p in (0, 1):
        assert np.array_equal(u64(out2[p]), (u64(out[p]) + r[p]).astype(np.uint64))


@pytest.mark.parametrize("producer", ["layernorm", "gelu"])
def test_producer_planes_feed_public_matmul(producer):
    """A LayerNorm block or GeLU chain writing its output as the next
    product's digit planes (sufhip_x_planes) gives the same shares as the
    product of its int64 output, and the same int64 output beside them."""
    M, K, N = 64, 96, 64
    x = pfss.host_normal_fixed(75, 1.0, 0.0, F, M * K)
    x0, x1 = _pair(x, 76)
    xin = (dev(x0), dev(x1))
    W = pfss.host_normal_fixed(77, 0.05, 0.0, F, K * N).view(np.int64).reshape(K, N)
    pm = layer.PublicMatmulTrunc(M, K, N, W, Dealer(8), STATE, F)
    say("producer planes: %s %dx%d -> %d" % (producer, M, K, N))
    if producer == "layernorm":
        blk = layer.LayerNormBlock(M, K, STATE, F, seed=31)
        assert blk.fusable()
    else:
        tab = tables.gelu_table(F)
        blk = layer.spline.SplineGate(M * K, tab[0], tab[1], STATE, F, seed=32, nonce=5)
    for t in blk.truncs():
        t.prepare()
    h = tuple(torch.empty(M * K, dtype=torch.int64, device="cuda") for _ in range(2))
    h2 = tuple(torch.empty(M * K, dtype=torch.int64, device="cuda") for _ in range(2))
    blk.eval2(xin, h)
    blk.eval2(xin, h2, planes=pm.x_planes())  # int64 output and planes
    for p in (0, 1):
        assert np.array_equal(u64(h[p]), u64(h2[p]))
    ref = tuple(torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    got = tuple(torch.empty(M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    pm.product2(h, out=ref)
    blk.eval2(xin, h2, planes=pm.x_planes(), write_out=False)
    pm.product2(None, out=got)
    for p in (0, 1):
        assert np.array_equal(u64(ref[p]), u64(got[p]))


def test_layernorm_reduces_product_slices():
    """A LayerNorm block over a public-weight product's unreduced k-slices
    (sufhip_matmul_public2_planes_partial, then sufhip_layernorm2 with
    in_slices: the reduction, the truncation and its residual addend in the
    block's launch) writes the same truncated product + residual and the same
    normalised shares as the product's own reduction followed by the block
    (the output projection and second LayerNorm of the layer, 128 x 768)."""
    M, K, N = 128, 768, 768
    say("layernorm over product slices %dx%dx%d" % (M, K, N))
    x = pfss.host_normal_fixed(91, 1.0, 0.0, F, M * K)
    xin = tuple(dev(v) for v in _pair(x, 92))
    W = pfss.host_normal_fixed(93, 0.05, 0.0, F, K * N).view(np.int64).reshape(K, N)
    res = tuple(dev(v) for v in _pair(pfss.host_normal_fixed(94, 1.0, 0.0, F, M * N), 95))
    pm = layer.PublicMatmulTrunc(M, K, N, W, Dealer(5), STATE, F)
    assert pm.slices() > 1
    ln = layer.LayerNormBlock(M, N, STATE, F, seed=33)
    assert ln.fusable()
    for t in pm.truncs() + ln.truncs():
        t.prepare()
    pair_ = lambda: tuple(torch.empty(M * N, dtype=torch.int64, device="cuda")  # noqa: E731
                          for _ in range(2))
    r_want, h_want, r_got, h_got = pair_(), pair_(), pair_(), pair_()
    pm.eval2(xin, r_want, add=res)  # X's planes stay in the product's workspace
    ln.eval2(r_want, h_want)
    for t in r_got + h_got:
        t.fill_(0x5a5a)
    pre = pm.eval2_slices(r_got, add=res)
    ln.eval2(None, h_got, pre=pre)
    torch.cuda.synchronize()
    for p in (0, 1):
        assert np.array_equal(u64(r_got[p]), u64(r_want[p])), ("r", p)
        assert np.array_equal(u64(h_got[p]), u64(h_want[p])), ("h", p)
    # Refused on the host: one slice, or a shape the product runs unsliced.
    a = ln.block_args(None, h_got, pre=(pre[0], 1, pre[2], pre[3]))
    with pytest.raises(native.SufHipError, match="in_slice_count"):
        native.call("sufhip_layernorm2", native.ctypes.byref(a), 0)
    small = layer.PublicMatmulTrunc(32, 64, 64, W[:64, :64], Dealer(6), STATE, F)
    assert small.slices() == 1
    with pytest.raises(native.SufHipError, match="one k-slice"):
        small.eval2_slices(pair_())


@pytest.mark.parametrize("rows,cols,gates,f,n", [
    (128, 768, 8, 12, 128 * 768),   # the layer's second LayerNorm gates in the first
    (128, 768, 5, 12, 128 * 3072),  # the MLP's gates in the second
    (128, 768, 12, 12, 1000),       # 24 jobs, the most one launch walks
    (64, 1536, 3, 14, 5000),        # 256-thread rows (the batched prepare first), f = 14
    (2080, 64, 2, 12, 4096),        # every CU holds a row: the walks come after
    (128, 768, 13, 12, 4096),       # 26 jobs: the batched prepare first
    (128, 768, 1, 20, 1 << 16),     # expansion launches: the batched prepare first
])
def test_layernorm_walks_later_gates(rows, cols, gates, f, n):
    """A fused LayerNorm launch that also walks other gates' key-only halves
    (sufhip_layernorm2's walk jobs, on the workgroups past the rows') writes
    the same normalised shares as the block alone and the same workspaces as
    the batched prepare, and the tables give the gates' shares.  Job sets the
    launch cannot walk go through the batched prepare first, same results."""
    from suf_amd.tasks import Trunc, prepare_batch
    say("layernorm with walks %dx%d, %d gates, f %d, n %d" % (rows, cols, gates, f, n))
    g = np.random.default_rng(rows + gates + f)
    m = rows * cols
    x = pfss.host_normal_fixed(101, 1.0, 0.0, F, m)
    xin = tuple(dev(v) for v in _pair(x, 102))
    ln = layer.LayerNormBlock(rows, cols, STATE, F, seed=35)
    assert ln.fusable()
    for t in ln.truncs():
        t.prepare()
    dealer = Dealer(22)
    trs = [Trunc(dealer, f, n, STATE) for _ in range(gates)]
    pair_ = lambda: tuple(torch.empty(m, dtype=torch.int64, device="cuda")  # noqa: E731
                          for _ in range(2))
    h_want, h_got = pair_(), pair_()
    ln.eval2(xin, h_want)
    for t in trs:
        for p in (0, 1):
            t.work[p].fill_(0x3c3c)
    for t in h_got:
        t.fill_(0x5a5a)
    ln.eval2(xin, h_got, walk=trs)
    torch.cuda.synchronize()
    got_work = [t.work[p].clone() for t in trs for p in (0, 1)]
    for t in trs:
        for p in (0, 1):
            t.work[p].fill_(0x3c3c)
    prepare_batch(trs)
    torch.cuda.synchronize()
    for p in (0, 1):
        assert np.array_equal(u64(h_got[p]), u64(h_want[p])), ("h", p)
    want_work = [t.work[p] for t in trs for p in (0, 1)]
    for i, (gw, ww) in enumerate(zip(got_work, want_work)):
        assert torch.equal(gw, ww), ("workspace", i)
    for t in (trs[0], trs[-1]):
        xs = g.integers(0, 2**40, n, dtype=np.uint64)
        out = (torch.empty(n, dtype=torch.int64, device="cuda"),
               torch.empty(n, dtype=torch.int64, device="cuda"))
        t.finish(dev(xs + np.uint64(t.mask)), out)
        assert np.array_equal(u64(out[0] + out[1]), xs >> np.uint64(f))


@pytest.mark.parametrize("rows,cols,slices", [(2080, 64, 5), (2080, 320, 3), (96, 1024, 2)])
def test_layernorm_in_slices_several_rows_per_workgroup(rows, cols, slices):
    """sufhip_layernorm2 over synthetic k-slices, with more rows than the
    launch has workgroups (2080 > 8 per CU: some workgroups take two rows)
    and with 2, 3 and 5 slices (groups of four and single slices): x = the
    truncation of the slices' open plus a residual, as the gate's own finish
    computes it, then the block, equal to the block over that x."""
    from suf_amd.tasks import Trunc
    say("layernorm in_slices %dx%d, %d slices" % (rows, cols, slices))
    n = rows * cols
    g = np.random.default_rng(rows + cols + slices)
    # Slice sums of a Q(f) value near 1: each party's slices are random but
    # sum to its share of x (x = x_0 + x_1 + r).
    x = pfss.host_normal_fixed(96, 1.0, 0.0, F, n).astype(np.uint64)
    parts = g.integers(0, 2**64, (slices, 2, n), dtype=np.uint64)
    x0 = g.integers(0, 2**64, n, dtype=np.uint64)
    parts[-1, 0] = (x0 - parts[:-1, 0].sum(axis=0, dtype=np.uint64)).astype(np.uint64)
    parts[-1, 1] = (x - x0 - parts[:-1, 1].sum(axis=0, dtype=np.uint64)).astype(np.uint64)
    dparts = dev(parts.reshape(-1))
    tr = Trunc(Dealer(40), F, n, STATE)
    tr.prepare()
    res = tuple(dev(v) for v in _pair(pfss.host_normal_fixed(97, 0.5, 0.0, F, n), 98))
    ln = layer.LayerNormBlock(rows, cols, STATE, F, seed=34)
    assert ln.fusable()
    for t in ln.truncs():
        t.prepare()
    pair_ = lambda: tuple(torch.empty(n, dtype=torch.int64, device="cuda")  # noqa: E731
                          for _ in range(2))
    r_want, h_want, r_got, h_got = pair_(), pair_(), pair_(), pair_()
    xhat = dev((x + np.uint64(tr.mask)).astype(np.uint64))
    tr.finish(xhat, r_want)
    for p in (0, 1):
        r_want[p].add_(res[p])
    ln.eval2(r_want, h_want)
    for t in r_got + h_got:
        t.fill_(0x5a5a)
    ln.eval2(None, h_got, pre=(dparts.data_ptr(), slices, tr.epilogue(r_got, res), tr.mask))
    torch.cuda.synchronize()
    for p in (0, 1):
        assert np.array_equal(u64(r_got[p]), u64(r_want[p])), ("r", p)
        assert np.array_equal(u64(h_got[p]), u64(h_want[p])), ("h", p)


@pytest.mark.parametrize("seq,d,heads", [(64, 128, 2), (128, 768, 12)])
def test_qkv_product_writes_attention_opens(seq, d, heads):
    """The QKV product writing the attention's three opens in its epilogue
    (sufhip_matmul_public2_planes_qkv) gives the same digit planes (Q_h - A
    with + A_0, K_h^T - B, V_h - B2) as the product's truncated output
    followed by the strided-view open-and-split launch."""
    say("qkv product -> attention opens seq=%d d=%d heads=%d" % (seq, d, heads))
    dealer = Dealer(7)
    x = pfss.host_normal_fixed(101, 1.0, 0.0, F, seq * d)
    xin = tuple(dev(v) for v in _pair(x, 102))
    W = pfss.host_normal_fixed(103, 0.05, 0.0, F, d * 3 * d).view(np.int64).reshape(d, 3 * d)
    pm = layer.PublicMatmulTrunc(seq, d, 3 * d, W, dealer, STATE, F)
    assert pm.slices() == 1
    attn = layer.AttentionCore(seq, d, heads, dealer, STATE, F)
    assert attn.mfma()
    pm.tr.prepare()
    qkv = tuple(torch.empty(seq * 3 * d, dtype=torch.int64, device="cuda") for _ in range(2))
    pm.eval2(xin, qkv)  # X's planes stay in the product's workspace
    tq, tp = attn.tri_qk, attn.tri_pv
    dh = d // heads
    planes = [tq.Dp, tq.Xp, tq.Ep, tp.Ep]
    layer.kb_open_split([(qkv, tq.A, tq.Dp, heads, seq, dh, 1, tq.Xp, tq.A[0], (0, dh, 3 * d, 1)),
                         (qkv, tq.B, tq.Ep, heads, dh, seq, 0, None, None, (d, dh, 1, 3 * d)),
                         (qkv, tp.B, tp.Ep, heads, seq, dh, 0, None, None,
                          (2 * d, dh, 3 * d, 1))])
    torch.cuda.synchronize()
    want = [t.clone() for t in planes]
    for t in planes:
        t.fill_(0x5a5a)  # every planes byte must be written
    pm.eval2_qkv(attn.qkv_opens())
    torch.cuda.synchronize()
    nbytes = native.load().sufhip_kb_planes_bytes(heads, seq, dh)
    for i, (g_, w_) in enumerate(zip(planes, want)):
        assert torch.equal(g_.view(torch.uint8)[:nbytes], w_.view(torch.uint8)[:nbytes]), i
    # Refused on the host: K^T's planes with the row-side layout.
    bad = attn.qkv_opens()
    bad.out[1].k_is_col = 1
    with pytest.raises(native.SufHipError, match="out\\[j\\]"):
        epi = pm.tr.epilogue((pm.zhat, pm.zhat))
        native.call("sufhip_matmul_public2_planes_qkv", pm.work.data_ptr(), seq, d, 3 * d,
                    pm.planes.data_ptr(), pm.digits, pm.tr.mask, native.ctypes.byref(epi),
                    native.ctypes.byref(bad), pm.work.data_ptr(), pm.work_bytes, 0)


def test_lin2_batch_matches_single_launches():
    """Four opens of different sizes in one launch equal four sufhip_lin2
    calls; a batch with a bad operand is refused on the host."""
    from suf_amd.tasks import lin2, lin2_batch, operand, term
    sizes = [1000, 1, 70000, 257]
    jobs, want, keep = [], [], []  # keep: the operands' tensors stay alive until the batch
    for k, n in enumerate(sizes):
        v = pfss.host_mt19937_64(80 + k, 3 * n).reshape(3, n)
        a = (dev(v[0]), dev(v[1]))
        b = (dev(v[2]), dev(v[2]))
        keep.append((a, b))
        x = operand(term(a), term(b, neg=True), const=k + 1)
        hat = torch.empty(n, dtype=torch.int64, device="cuda")
        ref = torch.empty(n, dtype=torch.int64, device="cuda")
        lin2(x, n, xhat=ref, mask=1000 + k)
        jobs.append((x, n, hat, 1000 + k))
        want.append(ref)
    say("lin2 batch %s" % sizes)
    lin2_batch(jobs)
    for (_, _, hat, _), ref in zip(jobs, want):
        assert np.array_equal(u64(hat), u64(ref))
    bad = term((dev(np.zeros(4, np.uint64)), dev(np.zeros(4, np.uint64))))  # 4 < n elements
    with pytest.raises(native.SufHipError):
        lin2_batch([(operand(bad), 1000, jobs[0][2], 0)])


@pytest.mark.parametrize("b,M,K,N", [
    (3, 32, 64, 48),     # VALU product (N not a multiple of 32)
    (3, 32, 64, 64),     # matrix cores
    (2, 64, 128, 32),    # matrix cores, PV-shaped
    (12, 128, 64, 128),  # matrix cores, the GPT-2 QK^T shape
])
def test_beaver_matmul2_batched_vs_oracle(b, M, K, N):
    X = pfss.host_normal_fixed(81, 1.0, 0.0, F, b * M * K).reshape(b, M, K)
    Y = pfss.host_normal_fixed(82, 1.0, 0.0, F, b * K * N).reshape(b, K, N)
    say("beaver matmul2 batched b=%d %dx%dx%d" % (b, M, K, N))
    tri = layer.BatchedTriples(Dealer(5), b, M, K, N)
    assert tri.mfma == (M % 32 == 0 and K % 32 == 0 and N % 32 == 0)
    A, B, C, A0, B0, C0 = tri.host
    A1, B1, C1 = A - A0, B - B0, C - C0
    x0 = pfss.host_mt19937_64(83, X.size).reshape(X.shape)
    y0 = pfss.host_mt19937_64(84, Y.size).reshape(Y.shape)
    D = ((x0 - A0) + (X - x0 - A1)).astype(np.uint64)
    E = ((y0 - B0) + (Y - y0 - B1)).astype(np.uint64)
    out = tuple(torch.empty(b * M * N, dtype=torch.int64, device="cuda") for _ in range(2))
    layer._beaver_batched(dev(D), dev(E), tri, b, M, K, N, out)
    g = [u64(out[0]).reshape(b, M, N), u64(out[1]).reshape(b, M, N)]
    for i in sorted({0, b - 1}):
        for p, (Ap, Bp, Cp) in enumerate(((A0, B0, C0), (A1, B1, C1))):
            o = ol.beaver_matmul(p, D[i], E[i], Ap[i], Bp[i], Cp[i], 1, M, K, N)
            assert np.array_equal(g[p][i].ravel(), np.asarray(o).ravel())
    rec = (g[0] + g[1]).astype(np.uint64)
    assert np.array_equal(rec, np.matmul(X, Y))
    if tri.mfma:  # the same shares from the VALU product
        wb = native.load().sufhip_beaver_matmul2_batched_work_bytes(b, M, K, N)
        work = torch.empty(max(2, (wb + 15) // 8), dtype=torch.int64, device="cuda")
        ref = tuple(torch.empty(b * M * N, dtype=torch.int64, device="cuda") for _ in range(2))
        Dd, Ed = dev(D), dev(E)
        native.call("sufhip_beaver_matmul2_batched", Dd.data_ptr(), Ed.data_ptr(),
                    tri.A[0].data_ptr(), tri.A[1].data_ptr(), tri.B[0].data_ptr(),
                    tri.B[1].data_ptr(), tri.C[0].data_ptr(), tri.C[1].data_ptr(), b, M, K, N,
                    ref[0].data_ptr(), ref[1].data_ptr(), work.data_ptr(), work.numel() * 8,
                    torch.cuda.current_stream().cuda_stream)
        for p in (0, 1):
            assert np.array_equal(u64(ref[p]), u64(out[p]))


@pytest.mark.parametrize("b,M,K,N", [
    (1, 32, 32, 32),      # one k-step: fewer operand pairs than pipeline stages
    (3, 64, 96, 32),      # 6 pairs: not a multiple of the stage count
    (2, 32, 160, 64),     # 10 pairs
    (1, 128, 768, 3072),  # the config-3 product
])
def test_beaver_balanced_form_equals_three_product_form(b, M, K, N):
    """With the planes of D + A_0 (Xp) each party's share takes two operand
    products per k-step; the shares equal the three-product form's (no Xp),
    and the oracle's for the small shapes."""
    say("beaver balanced form b=%d %dx%dx%d" % (b, M, K, N))
    tri = layer.BatchedTriples(Dealer(31), b, M, K, N)
    g = np.random.default_rng(b * 7 + K)
    D = g.integers(0, 2**64, b * M * K, dtype=np.uint64)
    E = g.integers(0, 2**64, b * K * N, dtype=np.uint64)
    D[:4] = [2**64 - 1, 2**63, 0x8080808080808080, 0x7F7F7F7F7F7F7F7F]
    layer.kb_split(tri.split_jobs(dev(D), dev(E)))
    outs = []
    for balanced in (True, False):
        a = tri.mfma_args()
        if not balanced:
            a.Xp = None
        out = tuple(torch.empty(b * M * N, dtype=torch.int64, device="cuda") for _ in range(2))
        a.out[0], a.out[1] = out[0].data_ptr(), out[1].data_ptr()
        native.call("sufhip_beaver_matmul2_mfma_ex", native.ctypes.byref(a), 0)
        outs.append([u64(o).reshape(b, M, N) for o in out])
    for p in (0, 1):
        assert np.array_equal(outs[0][p], outs[1][p]), p
    if b * M * K * N <= 1 << 20:
        A, B, C, A0, B0, C0 = tri.host
        for i in range(b):
            for p, (Ap, Bp, Cp) in enumerate(((A0, B0, C0), (A - A0, B - B0, C - C0))):
                o = ol.beaver_matmul(p, D.reshape(b, M, K)[i], E.reshape(b, K, N)[i], Ap[i],
                                     Bp[i], Cp[i], 1, M, K, N)
                assert np.array_equal(outs[0][p][i].ravel(), np.asarray(o).ravel()), (i, p)


@pytest.mark.parametrize("shape", [(1, 64, 96, 1), (2, 32, 64, 1), (1, 96, 64, 0)])
def test_split_planes_a0_are_planes_of_value_plus_a0(shape):
    """planes_a0 of a split and of an open-split job are the planes of the
    value + a0, written in the same launch (every byte)."""
    nb, r, c, kc = shape
    say("split planes_a0 %s" % (shape,))
    g = np.random.default_rng(11)
    n = nb * r * c
    src = dev(g.integers(0, 2**64, n, dtype=np.uint64))
    a0 = dev(g.integers(0, 2**64, n, dtype=np.uint64))
    a = tuple(dev(g.integers(0, 2**64, n, dtype=np.uint64)) for _ in range(2))
    bb = tuple(dev(g.integers(0, 2**64, n, dtype=np.uint64)) for _ in range(2))
    nbytes = native.load().sufhip_kb_planes_bytes(nb, r, c)
    for value, job in ((src, lambda pl, px: layer.kb_split([(src, pl, nb, r, c, kc, px, a0)])),
                       (a[0] + a[1] - bb[0] - bb[1],
                        lambda pl, px: layer.kb_open_split([(a, bb, pl, nb, r, c, kc, px, a0)]))):
        want, want_x = layer.kb_planes(nb, r, c), layer.kb_planes(nb, r, c)
        layer.kb_split([(value, want, nb, r, c, kc), (value + a0, want_x, nb, r, c, kc)])
        got, got_x = layer.kb_planes(nb, r, c), layer.kb_planes(nb, r, c)
        got.fill_(0x5a5a)
        got_x.fill_(0x5a5a)
        job(got, got_x)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.uint8)[:nbytes], want.view(torch.uint8)[:nbytes])
        assert torch.equal(got_x.view(torch.uint8)[:nbytes], want_x.view(torch.uint8)[:nbytes])
    with pytest.raises(native.SufHipError, match="planes_a0 and a0"):
        arr = (native.KbSplitJob * 1)()
        arr[0].src, arr[0].planes = src.data_ptr(), want.data_ptr()
        arr[0].batches, arr[0].rows, arr[0].cols, arr[0].k_is_col = nb, r, c, kc
        arr[0].planes_a0 = want_x.data_ptr()  # without a0
        native.call("sufhip_kb_split_batch", arr, 1, 0)


def test_beaver_trunc_merged_matches_separate_launches():
    """PV with the context's truncation and head merge folded into the
    product's launch (sufhip_beaver_matmul2_mfma_ex) gives the shares of the
    product, a gather and a truncation launch; its digit-plane output feeds
    the output projection like the merged shares do."""
    h, seq, dh = 4, 64, 32
    d = h * dh
    say("beaver trunc merged h=%d seq=%d dh=%d" % (h, seq, dh))
    tri = layer.BatchedTriples(Dealer(9), h, seq, seq, dh)
    assert tri.mfma
    tr = layer.Trunc(Dealer(10), F, seq * d, STATE)
    tr.prepare()
    P = pfss.host_normal_fixed(85, 0.3, 0.0, F, h * seq * seq).reshape(h, seq, seq)
    V = pfss.host_normal_fixed(86, 1.0, 0.0, F, h * seq * dh).reshape(h, seq, dh)
    A, B, C, A0, B0, C0 = tri.host
    D = (P - A).astype(np.uint64)
    E = (V - B).astype(np.uint64)
    Z = tuple(torch.empty(h * seq * dh, dtype=torch.int64, device="cuda") for _ in range(2))
    layer._beaver_batched(dev(D), dev(E), tri, h, seq, seq, dh, Z)
    mp = layer.attention_maps(seq, d, h)
    gc = layer.dev_i32(mp["gc"])
    ref = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    layer.lin2(layer.operand(layer.term(Z, index=gc)), seq * d, into=(tr, ref))
    W = pfss.host_normal_fixed(87, 0.05, 0.0, F, d * 64).view(np.int64).reshape(d, 64)
    pm = layer.PublicMatmulTrunc(seq, d, 64, W, Dealer(11), STATE, F)
    got = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    layer._beaver_trunc_merged(tri, tr, got, pm.x_planes())  # tri.Dp / Ep hold D, E
    for p in (0, 1):
        assert np.array_equal(u64(got[p]), u64(ref[p]))
    y_ref = tuple(torch.empty(seq * 64, dtype=torch.int64, device="cuda") for _ in range(2))
    y_got = tuple(torch.empty(seq * 64, dtype=torch.int64, device="cuda") for _ in range(2))
    pm.product2(None, out=y_got)
    pm.product2(ref, out=y_ref)
    for p in (0, 1):
        assert np.array_equal(u64(y_got[p]), u64(y_ref[p]))


def test_kb_split_rejects_bad_shapes():
    src = dev(np.zeros(48 * 64, np.uint64))
    planes = layer.kb_planes(1, 32, 64)
    with pytest.raises(native.SufHipError):
        layer.kb_split([(src, planes, 1, 48, 64, 1)])  # rows not a multiple of 32
    with pytest.raises(native.SufHipError):
        layer.kb_split([(src, planes, 1, 32, 64, 1)] * 9)  # more than 8 jobs
    assert native.load().sufhip_kb_planes_bytes(1, 40, 64) == 0


def _layer_case(seq, d, heads, ffn, seed):
    W = layer.synthetic_weights(d, ffn, F, seed)
    x = pfss.host_normal_fixed(seed + 1, 1.0, 0.0, F, seq * d)
    return W, x


@pytest.mark.parametrize("seq,d,heads", [(32, 64, 2), (64, 128, 4)])
def test_attention_core_reconstructs(seq, d, heads):
    qkv = pfss.host_normal_fixed(90 + seq, 1.0, 0.0, F, seq * 3 * d)
    q0, q1 = _pair(qkv, 91)
    say("attention core seq=%d d=%d heads=%d" % (seq, d, heads))
    at = layer.AttentionCore(seq, d, heads, Dealer(6), STATE, F)
    for t in at.truncs():
        t.prepare()
    tabs = _tabs()
    want, st = fp.attention(qkv, seq, d, heads, F, tabs["nexp"], tabs["recip"])
    shares = []
    for fused in (False, True):
        out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
        at.eval2((dev(q0), dev(q1)), out, fused=fused)
        if not fused:  # the one-launch softmax keeps the scores on chip
            sc = (u64(at.scores[0]) + u64(at.scores[1])).astype(np.uint64)
            assert np.array_equal(sc, st["scores"].view(np.uint64))
        rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
        assert np.array_equal(rec, want.view(np.uint64))
        shares.append((u64(out[0]), u64(out[1])))
    # Same dealer material: the fused path's shares equal the per-launch path's.
    assert np.array_equal(shares[0][0], shares[1][0])
    assert np.array_equal(shares[0][1], shares[1][1])


def test_layer_small_reconstructs():
    seq, d, heads, ffn = 32, 64, 2, 128
    W, x = _layer_case(seq, d, heads, ffn, 21)
    x0, x1 = _pair(x, 22)
    say("transformer layer small seq=%d d=%d heads=%d ffn=%d" % (seq, d, heads, ffn))
    ly = layer.TransformerLayer(STATE, W, seq, d, heads, ffn, F, seed=23, keep_intermediates=True)
    out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    ly.eval2((dev(x0), dev(x1)), out)
    want, st = fp.transformer_layer(x, W, seq, d, heads, ffn, F, _tabs(),
                                    tables.inv_len_qf(d), tables.eps_qf())
    for name, t in (("h1", ly.h1), ("qkv", ly.qkvs), ("ctx", ly.ctx), ("r1", ly.r1),
                    ("h2", ly.h2), ("u", ly.u), ("g", ly.g)):
        rec = (u64(t[0]) + u64(t[1])).astype(np.uint64)
        assert np.array_equal(rec, st[name].view(np.uint64).ravel()), name
    rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
    assert np.array_equal(rec, want.view(np.uint64))


def test_layer_config_shape_twice():
    seq, d, heads, ffn = 128, 768, 12, 3072
    W, x = _layer_case(seq, d, heads, ffn, 13)
    x0, x1 = _pair(x, 141)
    say("transformer layer config shape")
    ly = layer.TransformerLayer(STATE, W, seq, d, heads, ffn, F, seed=13)
    want, _ = fp.transformer_layer(x, W, seq, d, heads, ffn, F, _tabs(),
                                   tables.inv_len_qf(d), tables.eps_qf())
    xin = (dev(x0), dev(x1))
    out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    for _ in range(2):
        ly.eval2(xin, out)
        rec = (u64(out[0]) + u64(out[1])).astype(np.uint64)
        assert np.array_equal(rec, want.view(np.uint64))


@pytest.mark.parametrize("seq,d,heads,ffn", [(32, 64, 2, 128), (128, 768, 12, 3072)])
def test_layer_shares_equal_twoparty_oracle(seq, d, heads, ffn):
    """Both parties' shares of every stage and of the output equal the
    oracle's two-party composition of the same protocol steps (LayerNorm,
    public products with their truncation gates, per-head Beaver products,
    the softmax block, GeLU) on the same dealer material."""
    import twoparty_oracle as tp

    W, x = _layer_case(seq, d, heads, ffn, 31)
    x0, x1 = _pair(x, 32)
    say("transformer layer shares vs two-party oracle seq=%d d=%d heads=%d ffn=%d"
        % (seq, d, heads, ffn))
    ly = layer.TransformerLayer(STATE, W, seq, d, heads, ffn, F, seed=33, keep_intermediates=True)
    out = tuple(torch.empty(seq * d, dtype=torch.int64, device="cuda") for _ in range(2))
    ly.eval2((dev(x0), dev(x1)), out)
    torch.cuda.synchronize()
    want, st = tp.layer2(ol.Prg(STATE), ly, (x0, x1))
    for name, t in (("h1", ly.h1), ("qkv", ly.qkvs), ("ctx", ly.ctx), ("r1", ly.r1),
                    ("h2", ly.h2), ("u", ly.u), ("g", ly.g)):
        for p in (0, 1):
            assert np.array_equal(u64(t[p]), st[name][p]), (name, p)
    for p in (0, 1):
        assert np.array_equal(u64(out[p]), want[p]), p


def test_plane_outputs_reject_bad_layouts():
    """The digit-plane outputs and inputs are checked on the host: a plane
    layout that does not cover the open, a head-merged plane output without
    merge_heads, and unaligned X planes are refused before any launch."""
    x = (dev(np.zeros(64 * 64, np.uint64)), dev(np.zeros(64 * 64, np.uint64)))
    planes = layer.kb_planes(1, 64, 64)
    with pytest.raises(native.SufHipError):  # 64 x 64 planes for 32 x 64 elements
        layer.lin2_batch([(layer.operand(layer.term(x)), 32 * 64, None, 0,
                           (planes, 1, 64, 64, 1))])
    with pytest.raises(native.SufHipError):  # rows not a multiple of 32
        layer.lin2_batch([(layer.operand(layer.term(x)), 48 * 64, None, 0,
                           (planes, 1, 48, 64, 1))])
    tri = layer.BatchedTriples(Dealer(12), 2, 32, 32, 32)
    a = native.BeaverMfma2Args()
    a.Dp, a.Ep = tri.Dp.data_ptr(), tri.Ep.data_ptr()
    for p in (0, 1):
        a.Ap[p], a.Bp[p], a.C[p] = tri.Ap[p].data_ptr(), tri.Bp[p].data_ptr(), tri.C[p].data_ptr()
    out = tuple(torch.empty(2 * 32 * 32, dtype=torch.int64, device="cuda") for _ in range(2))
    a.batches, a.M, a.K, a.N = 2, 32, 32, 32
    a.out[0], a.out[1] = out[0].data_ptr(), out[1].data_ptr()
    a.out_planes.planes, a.out_planes.cols = planes.data_ptr(), 64  # without merge_heads
    with pytest.raises(native.SufHipError):
        native.call("sufhip_beaver_matmul2_mfma_ex", native.ctypes.byref(a), 0)
    W = np.ones((64, 32), np.int64)
    pm = layer.PublicMatmulTrunc(32, 64, 32, W, Dealer(13), STATE, F)
    with pytest.raises(native.SufHipError):  # X planes not 16-byte aligned
        native.call("sufhip_matmul_public2_planes", pm.work.data_ptr() + 8, 32, 64, 32,
                    pm.planes.data_ptr(), pm.digits, out[0].data_ptr(), out[1].data_ptr(), None,
                    0, None, pm.work.data_ptr(), pm.work_bytes, 0)


@pytest.mark.parametrize("shape", [(1, 64, 96, 1), (1, 96, 64, 0), (3, 32, 64, 0),
                                   (1, 1024, 2048, 0)])
def test_kb_open_split_matches_open_then_split(shape):
    """The open-and-split launch writes the same digit planes as the open
    a0 + a1 - b0 - b1 in u64 followed by the split, with and without b.  The
    last shape is large enough for 16 k per lane on the column side (the
    others take 4)."""
    nb, r, c, kc = shape
    print("[gpu-case] kb_open_split", shape, flush=True)
    g = np.random.default_rng(7)
    n = nb * r * c
    a = tuple(dev(g.integers(0, 2**63, n, dtype=np.uint64) * 2 + 1) for _ in range(2))
    b = tuple(dev(g.integers(0, 2**63, n, dtype=np.uint64)) for _ in range(2))
    for use_b in (True, False):
        opened = a[0] + a[1] - (b[0] + b[1] if use_b else 0)
        want = layer.kb_planes(nb, r, c)
        got = layer.kb_planes(nb, r, c)
        want.fill_(0)
        got.fill_(0x5a5a)  # every planes byte must be written
        layer.kb_split([(opened, want, nb, r, c, kc)])
        layer.kb_open_split([(a, b if use_b else None, got, nb, r, c, kc)])
        torch.cuda.synchronize()
        nbytes = native.load().sufhip_kb_planes_bytes(nb, r, c)
        assert torch.equal(got.view(torch.uint8)[:nbytes], want.view(torch.uint8)[:nbytes]), \
            (shape, use_b)
    with pytest.raises(native.SufHipError):  # rows not a multiple of 32
        layer.kb_open_split([(a, b, layer.kb_planes(1, 64, 64), 1, 48, 64, 1)])
    for one_sided in ((b[0], None), (None, b[1])):  # one share of b only
        arr = (native.KbOpenJob * 1)()
        arr[0].a[0], arr[0].a[1] = a[0].data_ptr(), a[1].data_ptr()
        arr[0].b[0] = one_sided[0].data_ptr() if one_sided[0] is not None else None
        arr[0].b[1] = one_sided[1].data_ptr() if one_sided[1] is not None else None
        arr[0].planes = layer.kb_planes(nb, r, c).data_ptr()
        arr[0].batches, arr[0].rows, arr[0].cols, arr[0].k_is_col = nb, r, c, kc
        with pytest.raises(native.SufHipError, match="both shares of b"):
            native.call("sufhip_kb_open_split_batch", arr, 1, 0)


@pytest.mark.parametrize("seq,d,heads", [(64, 128, 2), (128, 768, 12)])
def test_kb_open_split_strided_views_match_gathers(seq, d, heads):
    """The attention's three opens read through strided views of the QKV rows
    (Q_h - A with the planes of + A_0, K_h^T - B, V_h - B2) write the same
    planes as the opens of the index-map gathers (attention_maps) split
    plainly, in one launch."""
    print("[gpu-case] kb_open_split strided views", seq, d, heads, flush=True)
    dh = d // heads
    g = np.random.default_rng(9)
    qkv = tuple(dev(g.integers(0, 2**64, seq * 3 * d, dtype=np.uint64)) for _ in range(2))
    A = tuple(dev(g.integers(0, 2**64, heads * seq * dh, dtype=np.uint64)) for _ in range(2))
    B = tuple(dev(g.integers(0, 2**64, heads * dh * seq, dtype=np.uint64)) for _ in range(2))
    B2 = tuple(dev(g.integers(0, 2**64, heads * seq * dh, dtype=np.uint64)) for _ in range(2))
    mp = layer.attention_maps(seq, d, heads)
    shapes = [(heads, seq, dh, 1), (heads, dh, seq, 0), (heads, seq, dh, 0)]
    views = [(0, dh, 3 * d, 1), (d, dh, 1, 3 * d), (2 * d, dh, 3 * d, 1)]
    subs = [A, B, B2]
    got = [layer.kb_planes(*s[:3]) for s in shapes] + [layer.kb_planes(heads, seq, dh)]
    want = [layer.kb_planes(*s[:3]) for s in shapes] + [layer.kb_planes(heads, seq, dh)]
    for t in got:
        t.fill_(0x5a5a)  # every planes byte must be written
    jobs = []
    for i, (s, v, b) in enumerate(zip(shapes, views, subs)):
        extra = (got[3], A[0]) if i == 0 else (None, None)
        jobs.append((qkv, b, got[i], *s, *extra, v))
    layer.kb_open_split(jobs)
    for i, (s, key, b) in enumerate(zip(shapes, ("gq", "gk", "gv"), subs)):
        idx = torch.from_numpy(mp[key].astype(np.int64)).cuda()
        gathered = tuple(qkv[p][idx].contiguous() for p in (0, 1))
        extra = (want[3], A[0]) if i == 0 else ()
        layer.kb_open_split([(gathered, b, want[i], *s, *extra)])
    torch.cuda.synchronize()
    for i, (nb, r, c) in enumerate([s[:3] for s in shapes] + [(heads, seq, dh)]):
        nbytes = native.load().sufhip_kb_planes_bytes(nb, r, c)
        assert torch.equal(got[i].view(torch.uint8)[:nbytes], want[i].view(torch.uint8)[:nbytes]), i
    with pytest.raises(ValueError, match="outside"):  # the view's last element past qkv
        layer.kb_open_split([(qkv, B2, got[2], heads, seq, dh, 0, None, None,
                              (2 * d + 1, dh, 3 * d, 1))])


def test_kb_open_split_two_jobs_mixed():
    """One launch with two jobs: a column-side open with b (k_is_col 1) and a
    row-side open without b (k_is_col 0), each equal to its own open + split."""
    print("[gpu-case] kb_open_split two mixed jobs", flush=True)
    g = np.random.default_rng(8)
    specs = [(1, 64, 96, 1, True), (2, 32, 64, 0, False)]
    jobs, wants = [], []
    for nb, r, c, kc, use_b in specs:
        n = nb * r * c
        a = tuple(dev(g.integers(0, 2**64, n, dtype=np.uint64)) for _ in range(2))
        b = tuple(dev(g.integers(0, 2**64, n, dtype=np.uint64)) for _ in range(2))
        opened = a[0] + a[1] - (b[0] + b[1] if use_b else 0)
        want = layer.kb_planes(nb, r, c)
        want.fill_(0)
        layer.kb_split([(opened, want, nb, r, c, kc)])
        got = layer.kb_planes(nb, r, c)
        got.fill_(0x5a5a)
        jobs.append((a, b if use_b else None, got, nb, r, c, kc))
        wants.append((want, native.load().sufhip_kb_planes_bytes(nb, r, c)))
    layer.kb_open_split(jobs)
    torch.cuda.synchronize()
    for (want, nbytes), job in zip(wants, jobs):
        assert torch.equal(job[2].view(torch.uint8)[:nbytes], want.view(torch.uint8)[:nbytes])


@pytest.mark.parametrize("gates,f,n,big", [(1, 12, 4096, False), (2, 7, 100, False),
                                           (1, 14, 4096, False), (5, 12, 4096, False),
                                           (1, 20, 1 << 16, False), (1, 20, 4096, False),
                                           (1, 12, 128 * 3072, True)])
def test_kb_open_split_prepare_matches_separate_calls(gates, f, n, big):
    """The opens with the truncations' key-only walks in the same launch
    (sufhip_kb_open_split_prepare) write the same digit planes as the opens
    alone and the same workspaces as the batched prepare.  One or two table
    gates run in the one launch; f = 14 (walks past three quarters of a walk
    workgroup per CU), five gates (ten jobs, above eight), f = 20 with 2^16
    points (expansion launches) and f = 20 with 4096 points (a depth-12
    frontier, not a table) take the prepare's own launches first.  big: the
    matmul gate's shapes (D 128 x 768 with the planes of + A_0, E 768 x 3072),
    whose E goes by LDS tiles beside the walks."""
    from suf_amd.tasks import Trunc, prepare_batch
    print("[gpu-case] kb_open_split_prepare", gates, f, n, big, flush=True)
    g = np.random.default_rng(11)
    dealer = Dealer(21)
    trs = [Trunc(dealer, f, n, STATE) for _ in range(gates)]
    specs = [(1, 128, 768, 1, True), (1, 768, 3072, 0, True)] if big else \
        [(1, 64, 96, 1, True), (2, 32, 64, 0, False)]
    jobs, got_planes, want_planes = [], [], []
    for nb, r, c, kc, use_b in specs:
        m = nb * r * c
        a = tuple(dev(g.integers(0, 2**64, m, dtype=np.uint64)) for _ in range(2))
        b = tuple(dev(g.integers(0, 2**64, m, dtype=np.uint64)) for _ in range(2)) if use_b else None
        got_planes.append(layer.kb_planes(nb, r, c))
        want_planes.append(layer.kb_planes(nb, r, c))
        got_planes[-1].fill_(0x5a5a)  # every planes byte must be written
        want_planes[-1].fill_(0)
        jobs.append((a, b, nb, r, c, kc))
    for t in trs:
        for p in (0, 1):
            t.work[p].fill_(0x3c3c)
    layer.kb_open_split([(a, b, pl, nb, r, c, kc) for (a, b, nb, r, c, kc), pl
                         in zip(jobs, got_planes)], prepare=trs)
    torch.cuda.synchronize()
    got_work = [t.work[p].clone() for t in trs for p in (0, 1)]
    for t in trs:
        for p in (0, 1):
            t.work[p].fill_(0x3c3c)
    prepare_batch(trs)
    layer.kb_open_split([(a, b, pl, nb, r, c, kc) for (a, b, nb, r, c, kc), pl
                         in zip(jobs, want_planes)])
    torch.cuda.synchronize()
    want_work = [t.work[p] for t in trs for p in (0, 1)]
    for i, (gw, ww) in enumerate(zip(got_work, want_work)):
        assert torch.equal(gw, ww), ("workspace", i)
    for (a, b, nb, r, c, kc), gp, wp in zip(jobs, got_planes, want_planes):
        nbytes = native.load().sufhip_kb_planes_bytes(nb, r, c)
        assert torch.equal(gp.view(torch.uint8)[:nbytes], wp.view(torch.uint8)[:nbytes])
    # The tables give the gate's shares: x >> f after the finish (one gate).
    t = trs[0]
    x = g.integers(0, 2**40, n, dtype=np.uint64)
    xh = dev(x + np.uint64(t.mask))
    out = (torch.empty(n, dtype=torch.int64, device="cuda"),
           torch.empty(n, dtype=torch.int64, device="cuda"))
    t.finish(xh, out)
    assert np.array_equal(u64(out[0] + out[1]), x >> np.uint64(f))


@pytest.mark.parametrize("shape", [(1, 64, 96, 1), (2, 96, 64, 0), (3, 32, 64, 0)])
def test_lin2_batch_planes_match_open_then_split(shape):
    """lin2_batch's digit-plane output of an open (row-side layouts written in
    16-row runs, column-side element by element; with the planes of open + a0
    beside them) equals the open x0 + x1 + mask followed by the split."""
    nb, r, c, kc = shape
    print("[gpu-case] lin2_batch planes", shape, flush=True)
    g = np.random.default_rng(9)
    n = nb * r * c
    x = tuple(dev(g.integers(0, 2**64, n, dtype=np.uint64)) for _ in range(2))
    a0 = dev(g.integers(0, 2**64, n, dtype=np.uint64))
    mask = int(g.integers(0, 2**63)) * 2 + 1
    opened = x[0] + x[1] + torch.tensor(np.uint64(mask).view(np.int64), device="cuda")
    want = layer.kb_planes(nb, r, c)
    want_x = layer.kb_planes(nb, r, c)
    layer.kb_split([(opened, want, nb, r, c, kc), (opened + a0, want_x, nb, r, c, kc)])
    got = layer.kb_planes(nb, r, c)
    got_x = layer.kb_planes(nb, r, c)
    got.fill_(0x5a5a)
    got_x.fill_(0x5a5a)
    xhat = torch.empty(n, dtype=torch.int64, device="cuda")
    layer.lin2_batch([(layer.operand(layer.term(x)), n, xhat, mask,
                       (got, nb, r, c, kc, got_x, a0))])
    torch.cuda.synchronize()
    nbytes = native.load().sufhip_kb_planes_bytes(nb, r, c)
    assert torch.equal(xhat, opened)
    assert torch.equal(got.view(torch.uint8)[:nbytes], want.view(torch.uint8)[:nbytes])
    assert torch.equal(got_x.view(torch.uint8)[:nbytes], want_x.view(torch.uint8)[:nbytes])
