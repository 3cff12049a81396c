"""Host-side pieces of the spline gate (no GPU): the rotated interval-LUT
geometry returns the right piece's coefficients through the oracle LUT for
every mask, and the two-party step ABI struct matches its C layout."""
import ctypes
import os
import subprocess
import tempfile

import numpy as np
import pytest

import fixed_point as fp
import oracle_lib as ol
from suf_amd import native, spline

F = 12


def _lut_blob(party, cuts, payload, k):
    lib = native.load()
    kb = lib.sufhip_interval_lut_key_bytes(k, 4)
    seed16 = ctypes.create_string_buffer(16)
    lib.sufhip_seed_from_id(1, spline.LUT_TWEAK, seed16)
    blob = np.zeros(kb, dtype=np.uint8)
    native.call("sufhip_interval_lut_build_key", party, 1, 64, 4, cuts.ctypes.data, k,
                payload.ctypes.data, seed16, blob.ctypes.data)
    return blob, kb


@pytest.mark.parametrize("r_in", [0, 1, 12345 << F, (1 << 63) + 17, spline.M64,
                                  (1 << 64) - (8 << F), 8 << F])
def test_rotated_lut_selects_the_piece(r_in):
    alpha, coeffs = spline.spline_spec(F, seed=6)
    cuts, payload, k = spline.rotated_lut(alpha, coeffs, r_in)
    assert cuts[-1] == 0 and cuts[0] == 0 and np.all(np.diff(cuts[:-1].astype(object)) > 0)
    xs = [0, 1, (1 << F) - 1, 1 << F, (8 << F) - 1, 8 << F, (1 << 63) - 1, 1 << 63,
          (1 << 64) - (8 << F) - 1, (1 << 64) - (8 << F), spline.M64]
    rng = np.random.default_rng(r_in & 0xffff)
    xs += [int(v) for v in rng.integers(0, 1 << 64, 200, dtype=np.uint64)]
    x = np.array(xs, dtype=np.uint64)
    xhat = (x + np.uint64(r_in)).astype(np.uint64)
    b0, kb = _lut_blob(0, cuts, payload, k)
    b1, _ = _lut_blob(1, cuts, payload, k)
    rec = (ol.lut_eval(b0, kb, 1, xhat, 4) + ol.lut_eval(b1, kb, 1, xhat, 4)).astype(np.uint64)
    piece = np.searchsorted(alpha, x, side="right") - 1
    assert np.array_equal(rec.reshape(-1, 4), coeffs[piece].view(np.uint64))


def test_spline_closed_form_matches_python_ints():
    alpha, coeffs = spline.spline_spec(F, seed=6)
    rng = np.random.default_rng(2)
    x = np.array([int(v) & spline.M64 for v in rng.integers(-(8 << F), 8 << F, 300)],
                 dtype=np.uint64)
    got = fp.spline_closed_form(alpha, coeffs, x, F)
    for xi, gi in zip(x, got):
        xs = int(xi) - (1 << 64) if int(xi) >> 63 else int(xi)
        piece = int(np.searchsorted(alpha, xi, side="right")) - 1
        c0, c1, c2, c3 = (int(v) for v in coeffs[piece])
        p = (c3 * xs + (c2 << F)) * xs
        r = ((p >> F) + (c1 << F)) * xs
        assert int(gi) == ((r >> (2 * F)) + c0) & spline.M64


def test_mul2_args_layout_matches_c():
    src = r'''
#include <stdio.h>
#include <stddef.h>
#include "suf_hip.h"
#define O(f) printf("%s %zu\n", #f, offsetof(sufhip_mul2_args, f));
int main(void) {
  printf("size %zu\n", sizeof(sufhip_mul2_args));
  O(u) O(u_stride) O(u_off) O(u_add) O(u_add_stride) O(u_add_off) O(u_add_shift) O(v)
  O(triples) O(z_add) O(z_add_stride) O(z_add_off) O(z_add_shift) O(z) O(zhat) O(open_mask)
  return 0;
}
'''
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        exe = os.path.join(d, "l")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I" + os.path.join(ol.ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    want = dict((l.split()[0], int(l.split()[1])) for l in out.splitlines())
    assert want.pop("size") == ctypes.sizeof(native.Mul2Args)
    for name, off in want.items():
        assert getattr(native.Mul2Args, name).offset == off, name


def _c_offsets(struct, fields):
    src = "#include <stdio.h>\n#include <stddef.h>\n#include \"suf_hip.h\"\nint main(void) {\n"
    src += '  printf("size %%zu\\n", sizeof(%s));\n' % struct
    for f in fields:
        src += '  printf("%s %%zu\\n", offsetof(%s, %s));\n' % (f, struct, f)
    src += "  return 0;\n}\n"
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "l.c")
        exe = os.path.join(d, "l")
        open(c, "w").write(src)
        subprocess.run(["gcc", "-I" + os.path.join(ol.ROOT, "include"), c, "-o", exe], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    return dict((l.split()[0], int(l.split()[1])) for l in out.splitlines())


@pytest.mark.parametrize("struct,cls", [("sufhip_composite_bool_args", "CompositeBoolArgs"),
                                        ("sufhip_stage_seg", "StageSeg"),
                                        ("sufhip_open_req", "OpenReq"),
                                        ("sufhip_kb_planes", "KbPlanes"),
                                        ("sufhip_kb_split_job", "KbSplitJob"),
                                        ("sufhip_kb_open_job", "KbOpenJob"),
                                        ("sufhip_beaver_mfma2_args", "BeaverMfma2Args"),
                                        ("sufhip_lin2_job", "Lin2Job")])
def test_composite_struct_layouts_match_c(struct, cls):
    k = getattr(native, cls)
    want = _c_offsets(struct, [f[0] for f in k._fields_])
    assert want.pop("size") == ctypes.sizeof(k)
    for name, off in want.items():
        assert getattr(k, name).offset == off, name
