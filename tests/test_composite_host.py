"""The composite gate's dealer compilation (suf_amd.composite.compile_bools:
mask rewrite, x^ segments, postfix programs) and the two-party network
oracle (tests/twoparty_oracle.composite_bool2), on the CPU: plaintext query
and cut bits at x^ = x + r_in, XOR-split with random shares, through the
oracle network with random triples, must reconstruct to the reference's SUF
evaluation (oracle/suf_ref.py) for masks that make pieces wrap, land on
boundaries, or vanish."""
import types

import numpy as np
import pytest
import torch

import composite_specs as cs
import suf_ref
import twoparty_oracle as tp
from suf_amd import composite, native

M64 = (1 << 64) - 1


def _gate(spec, r_in, n, g):
    queries, wraps, segs, prog, offs, ands = composite.compile_bools(spec, r_in)
    ell = len(spec["pieces"][0]["bools"])
    C = len(segs) - 1
    T = (2 * C - 1 if C > 0 else 0) + 2 * (C + 1) * ell
    w = g.integers(0, 2**64, (5, T, n), dtype=np.uint64)
    a, b, a0, b0, c0 = w
    c = a * b
    tri = [np.stack([a0, b0, c0], axis=1), np.stack([a - a0, b - b0, c - c0], axis=1)]
    if ands:
        bits = g.integers(0, 2, (5, ands, n), dtype=np.uint8)
        A, Bb, a0, b0, c0 = bits
        Cc = A & Bb
        pack = lambda x, y, z: (x | (y << 1) | (z << 2)).astype(np.uint8)  # noqa: E731
        bt = [torch.from_numpy(pack(a0, b0, c0).ravel()),
              torch.from_numpy(pack(A ^ a0, Bb ^ b0, Cc ^ c0).ravel())]
    else:
        bt = [None, None]
    w0 = g.integers(0, 2**64, len(wraps), dtype=np.uint64)
    return types.SimpleNamespace(
        n=n, cuts=[s for s, _ in segs[1:]], ell=ell, T=T, and_count=ands, prog=prog,
        prog_off=offs, queries=queries, segs=segs,
        tri=[torch.from_numpy(t.view(np.int64).ravel().copy()) for t in tri], bit_tri=bt,
        wrap_share=[w0, (np.array(wraps, np.uint64) - w0).astype(np.uint64)])


@pytest.mark.parametrize("spec", [cs.MIXED, cs.DRELU], ids=["mixed", "drelu"])
@pytest.mark.parametrize("r_in", [0, 1, 12345, (1 << 63) + 7, M64, (1 << 64) - (1 << 62),
                                  (1 << 62) + 4096])
def test_compiled_network_reconstructs_suf(spec, r_in):
    g = np.random.default_rng(r_in % 1000 + len(spec["pieces"]))
    n = 3000
    x = g.integers(0, 2**64, n, dtype=np.uint64)
    x[:12] = [0, 999, 1000, 2047, 2048, (1 << 62) - 1, 1 << 62, (1 << 63) - 5000, (1 << 63) - 1,
              1 << 63, (1 << 63) + (1 << 62), M64]
    x[12:800] = g.integers(-5000, 5000, 788).astype(np.int64).view(np.uint64)
    gate = _gate(spec, r_in, n, g)
    xhat = (x + np.uint64(r_in)).astype(np.uint64)

    def shares(bit):
        s0 = g.integers(0, 2, n, dtype=np.uint8)
        return s0, (s0 ^ bit.astype(np.uint8))

    pred = [np.zeros((len(gate.queries), n), np.uint8) for _ in range(2)]
    for q, (bits, theta) in enumerate(gate.queries):
        m = np.uint64(M64 if bits >= 64 else (1 << bits) - 1)
        pred[0][q], pred[1][q] = shares((xhat & m) < np.uint64(theta))
    cut = [np.zeros((len(gate.cuts), n), np.uint8) for _ in range(2)]
    for k, c in enumerate(gate.cuts):
        cut[0][k], cut[1][k] = shares(xhat < np.uint64(c))
    out = tp.composite_bool2(gate, pred, cut)
    rec = (out[0] + out[1]).astype(np.uint64)
    _, bools, _ = suf_ref.eval_suf(spec, x)
    assert np.array_equal(rec, bools.astype(np.uint64))


def test_segments_cover_the_ring_once():
    for r in (0, 5, (1 << 63), M64, (1 << 62) * 3):
        segs = composite.segments(np.array(cs.MIXED["alpha"], np.uint64), r)
        starts = [s for s, _ in segs]
        assert starts[0] == 0 and starts == sorted(set(starts))
        # Every x lands in the segment of its own piece.
        x = np.array([0, 1, (1 << 62) - 1, 1 << 62, (1 << 63) + 9, M64], np.uint64)
        xhat = (x + np.uint64(r)).astype(np.uint64)
        seg = np.searchsorted(np.array(starts, np.uint64), xhat, side="right") - 1
        piece = suf_ref.piece_index(cs.MIXED["alpha"], x)
        assert [segs[k][1] for k in seg] == list(piece)


def test_program_encoding():
    prog = composite.postfix(("xor", ("and", ("q", 2), ("not", ("w", 1))), ("const", 1)), [])
    assert prog == [native.BOOL_VAR | 2 << 4, native.BOOL_WRAP | 1 << 4, native.BOOL_NOT,
                    native.BOOL_AND, native.BOOL_CONST | 1 << 4, native.BOOL_XOR]
