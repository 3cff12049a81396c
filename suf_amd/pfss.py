"""Python host layer over the C ABI for device-resident batches.

torch supplies device memory and the current stream only; every computation
runs in libsuf_hip.so.  u64 ring values are carried in torch.int64 tensors
(same bits).  Names follow the reference's backend operations
(include/proto/myl7_fss_backend.hpp, include/proto/backend_gpu.hpp).
"""
import contextlib

import torch

from . import native

PRG_STATE_BYTES = 128


@contextlib.contextmanager
def keystream_per_party(on=True):
    """Within the block, every two-party LUT launch computes each party's
    keystream from its own blob (sufhip_set_keystream_per_party): the same
    shares, the cost of two parties in separate processes.  Launches (and
    graphs) issued inside keep that policy."""
    prev = native.load().sufhip_keystream_per_party()
    native.call("sufhip_set_keystream_per_party", 1 if on else 0)
    try:
        yield
    finally:
        native.call("sufhip_set_keystream_per_party", prev)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _ptr(t):
    return t.data_ptr() if t is not None else None


def _state_buf(prg_state):
    b = bytes(prg_state)
    if len(b) != PRG_STATE_BYTES:
        raise ValueError("prg_state must be %d bytes" % PRG_STATE_BYTES)
    return native.ctypes.create_string_buffer(b, len(b))


def dcf_key_bytes(in_bits, payload_len):
    return native.load().sufhip_dcf_key_bytes(in_bits, payload_len)


def dcf_gen(group, in_bits, prg_state, alpha, payload, seeds, payload_broadcast=True):
    """Batched myl7 DCF keygen on the device.

    alpha: int64[N]; payload: uint8[payload_len] (broadcast) or uint8[N, payload_len];
    seeds: uint8[N, chunks*32].  Returns (keys0, keys1): uint8[N, key_bytes].
    """
    n = alpha.numel()
    plen = payload.shape[-1]
    kb = dcf_key_bytes(in_bits, plen)
    if kb == 0:
        raise native.SufHipError("dcf_gen: bad (in_bits, payload_len)")
    chunks = (plen + 15) // 16
    if seeds.numel() != n * chunks * 32:
        raise ValueError("seeds must hold N * chunks * 32 bytes")
    k0 = torch.empty((n, kb), dtype=torch.uint8, device=alpha.device)
    k1 = torch.empty((n, kb), dtype=torch.uint8, device=alpha.device)
    st = _state_buf(prg_state)
    native.call("sufhip_dcf_gen", group, in_bits, st, _ptr(alpha), _ptr(payload), plen,
                1 if payload_broadcast else 0, _ptr(seeds), n, _ptr(k0), _ptr(k1), _stream())
    return k0, k1


def dcf_eval(group, in_bits, payload_len, prg_state, keys, xs, out_mode=native.DCF_OUT_BIT,
             out_bytes=1, broadcast=False, out=None):
    """One party's DCF shares at xs (int64[N]).  keys: uint8[N, key_bytes] or one key."""
    n = xs.numel()
    kb = keys.shape[-1]
    if out is None:
        if out_mode == native.DCF_OUT_BIT:
            out = torch.empty(n, dtype=torch.uint8, device=xs.device)
        elif out_mode == native.DCF_OUT_BYTES:
            out = torch.empty((n, out_bytes), dtype=torch.uint8, device=xs.device)
        else:
            out = torch.empty((n + 63) // 64, dtype=torch.int64, device=xs.device)
    st = _state_buf(prg_state)
    native.call("sufhip_dcf_eval", group, in_bits, payload_len, st, _ptr(keys), kb,
                1 if broadcast else 0, _ptr(xs), n, out_mode, out_bytes, _ptr(out), _stream())
    return out


def trunc_key_bytes(kind, frac_bits):
    return native.load().sufhip_trunc_key_bytes(kind, frac_bits)


def trunc_gen(kind, frac_bits, prg_state, rnd, device="cuda"):
    """Dealer keys of one truncation gate.  rnd: 19 host u64 words (numpy).
    Returns (key0, key1): uint8[key_bytes] device tensors (8-byte aligned)."""
    import numpy as np

    rnd = np.ascontiguousarray(rnd, dtype=np.uint64)
    if rnd.size != native.TRUNC_RAND_WORDS:
        raise ValueError("rnd must hold %d words" % native.TRUNC_RAND_WORDS)
    kb = trunc_key_bytes(kind, frac_bits)
    if kb == 0:
        raise native.SufHipError("trunc_gen: bad (kind, frac_bits)")
    k0 = torch.empty(kb // 8, dtype=torch.int64, device=device).view(torch.uint8)
    k1 = torch.empty(kb // 8, dtype=torch.int64, device=device).view(torch.uint8)
    native.call("sufhip_trunc_gen", kind, frac_bits, _state_buf(prg_state), rnd.ctypes.data,
                _ptr(k0), _ptr(k1), _stream())
    return k0, k1


def trunc_eval(kind, frac_bits, prg_state, key, xhat, out=None, work=None):
    """One party's truncated shares given the public masked inputs xhat (int64[N])."""
    n = xhat.numel()
    if out is None:
        out = torch.empty(n, dtype=torch.int64, device=xhat.device)
    wb = native.load().sufhip_trunc_work_bytes(frac_bits, n)
    if work is None and wb:
        work = torch.empty((wb + 7) // 8, dtype=torch.int64, device=xhat.device)
    native.call("sufhip_trunc_eval", kind, frac_bits, _state_buf(prg_state), _ptr(key),
                key.numel(), _ptr(xhat), n, _ptr(out), _ptr(work),
                work.numel() * 8 if work is not None else 0, _stream())
    return out


def aes128_ctr(round_keys, ctr_lo, ctr_hi, blocks, device="cuda", bitsliced=False, out=None):
    """AES-128-CTR keystream blocks (the LDS T-table kernel, or the bitsliced
    one when bitsliced is true); out: optional uint8 device buffer of
    blocks * 16 bytes."""
    if out is None:
        out = torch.empty(blocks * 16, dtype=torch.uint8, device=device)
    rk = native.ctypes.create_string_buffer(bytes(round_keys), 176)
    native.call("sufhip_aes128_ctr_bitsliced" if bitsliced else "sufhip_aes128_ctr", _ptr(out),
                rk, ctr_lo, ctr_hi, blocks, _stream())
    return out


def prg_mmo(prg_state, seeds, out_blocks=4):
    n = seeds.numel() // 16
    out = torch.empty(n * 16 * out_blocks, dtype=torch.uint8, device=seeds.device)
    st = _state_buf(prg_state)
    native.call("sufhip_prg_mmo", st, _ptr(seeds), n, out_blocks, _ptr(out), _stream())
    return out


def host_mt19937_64(seed, n):
    import numpy as np

    out = np.empty(n, dtype=np.uint64)
    native.call("sufhip_host_mt19937_64", seed, out.ctypes.data, n)
    return out


def host_normal_fixed(seed, sigma, clip, frac_bits, n):
    import numpy as np

    out = np.empty(n, dtype=np.uint64)
    native.call("sufhip_host_normal_fixed", seed, sigma, clip, frac_bits, out.ctypes.data, n)
    return out
