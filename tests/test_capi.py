"""C-ABI checks that need no GPU: the library loads, exports every symbol the
header declares, validates arguments before touching the device, and its
host helpers agree with the oracle."""
import ctypes
import subprocess

import numpy as np
import pytest

import oracle_lib as ol
from suf_amd import native


def test_exports_every_header_symbol():
    lib = native.load()
    syms = native.header_symbols()
    assert len(syms) >= 20
    out = subprocess.run(["nm", "-D", "--defined-only", native.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if l.strip()}
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    for s in syms:
        assert hasattr(lib, s)
        assert s in native._SIGS, "no ctypes signature for %s" % s


def test_abi_version():
    assert native.load().sufhip_abi_version() == 1


@pytest.mark.parametrize("in_bits,plen", [(64, 1), (64, 8), (13, 1), (12, 20), (1, 16), (64, 300)])
def test_key_bytes_match_oracle(in_bits, plen):
    assert native.load().sufhip_dcf_key_bytes(in_bits, plen) == ol.myl7_key_bytes(in_bits, plen)


@pytest.mark.parametrize("kind", [0, 1, 2])
@pytest.mark.parametrize("f", [1, 12, 24, 62])
def test_trunc_key_bytes_match_oracle(kind, f):
    lib = native.load()
    assert lib.sufhip_trunc_key_bytes(kind, f) == ol.trunc_key_bytes(kind, f) > 0
    assert lib.sufhip_trunc_key_bytes(kind, 0) == 0 == lib.sufhip_trunc_key_bytes(kind, 63)
    assert lib.sufhip_trunc_key_bytes(3, f) == 0


def test_trunc_workspace_sizes():
    lib = native.load()
    # Frontier depth: d = f for f <= 14 (full-domain table), else
    # d = min(f, max(floor(log2 n) - 1, 12), 22); 32 bytes per node, 2^d nodes
    # plus 2^(d-1) when levels beyond 12 are expanded; nothing for n = 0.
    assert lib.sufhip_trunc_work_bytes(12, 1 << 20) == 32 << 12
    assert lib.sufhip_trunc_work_bytes(12, 31) == 32 << 12
    assert lib.sufhip_trunc_work_bytes(13, 128) == 32 * ((1 << 13) + (1 << 12))
    assert lib.sufhip_trunc_work_bytes(24, 1 << 20) == 32 * ((1 << 19) + (1 << 18))
    assert lib.sufhip_trunc_work_bytes(24, 3000) == 32 << 12
    assert lib.sufhip_trunc_work_bytes(24, 128) == 32 << 12
    assert lib.sufhip_trunc_work_bytes(40, 1 << 30) == 32 * ((1 << 22) + (1 << 21))
    assert lib.sufhip_trunc_work_bytes(12, 0) == 0


def test_key_bytes_rejects_bad_geometry():
    lib = native.load()
    assert lib.sufhip_dcf_key_bytes(0, 1) == 0
    assert lib.sufhip_dcf_key_bytes(65, 1) == 0
    assert lib.sufhip_dcf_key_bytes(64, 0) == 0
    assert lib.sufhip_dcf_key_bytes(64, 256 * 16) == 0


def test_invalid_arguments_fail_before_device_work():
    lib = native.load()
    st = ctypes.create_string_buffer(128)
    # in_bits out of range
    rc = lib.sufhip_dcf_eval(0, 65, 1, st, 1, 2152, 0, 1, 4, 0, 1, 1, None)
    assert rc == native.OK - 1
    assert b"in_bits" in lib.sufhip_last_error()
    # key_bytes inconsistent with (in_bits, payload_len)
    rc = lib.sufhip_dcf_eval(0, 64, 1, st, 1, 2151, 0, 1, 4, 0, 1, 1, None)
    assert rc == -1 and b"key_bytes" in lib.sufhip_last_error()
    # unknown output mode
    rc = lib.sufhip_dcf_eval(0, 64, 1, st, 1, 2152, 0, 1, 4, 9, 1, 1, None)
    assert rc == -1 and b"out_mode" in lib.sufhip_last_error()
    # null device pointers
    rc = lib.sufhip_dcf_eval(0, 64, 1, st, None, 2152, 0, 1, 4, 0, 1, 1, None)
    assert rc == -1 and b"null" in lib.sufhip_last_error()
    # n == 0 is a successful no-op, as for the reference launchers
    assert lib.sufhip_dcf_eval(0, 64, 1, st, None, 2152, 0, None, 0, 0, 1, None, None) == 0
    rc = lib.sufhip_dcf_gen(2, 64, st, 1, 1, 1, 1, 1, 4, 1, 1, None)
    assert rc == -1 and b"group" in lib.sufhip_last_error()


def test_host_mt19937_matches_oracle():
    out = np.empty(1000, dtype=np.uint64)
    native.call("sufhip_host_mt19937_64", 42, out.ctypes.data, 1000)
    assert np.array_equal(out, ol.mt64(42, 1000))
    big = np.empty(10000, dtype=np.uint64)
    native.call("sufhip_host_mt19937_64", 5489, big.ctypes.data, 10000)
    assert int(big[-1]) == 9981545732273789042


def test_host_normal_fixed_statistics():
    n = 200000
    out = np.empty(n, dtype=np.uint64)
    native.call("sufhip_host_normal_fixed", 2, 1.0, 0.0, 12, out.ctypes.data, n)
    v = out.view(np.int64).astype(np.float64) / 4096.0
    assert abs(v.mean()) < 0.01
    assert abs(v.std() - 1.0) < 0.01
    clipped = np.empty(n, dtype=np.uint64)
    native.call("sufhip_host_normal_fixed", 5, 3.0, 8.0, 12, clipped.ctypes.data, n)
    c = clipped.view(np.int64)
    assert c.max() <= 8 * 4096 and c.min() >= -8 * 4096
    # Deterministic for a seed.
    again = np.empty(n, dtype=np.uint64)
    native.call("sufhip_host_normal_fixed", 2, 1.0, 0.0, 12, again.ctypes.data, n)
    assert np.array_equal(out, again)
