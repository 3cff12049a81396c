"""Composite party-key tapes for the Python host side.

write_composite_tape / read_composite_tape produce and parse the byte format
of gates::write_composite_tape / read_composite_tape
(include/gates/composite_fss.hpp:2458-2641), the same format as the C++ host
side's suf_hip::write_composite_tape (include/suf_hip/tape.hpp).  Fields, in
tape order, all little-endian:

  r_in_share u64 | r_in_share_vec [u32 n][u64 x n] | r_out_share [u32][u64..]
  | wrap_share [u32][u64..] | r_hi_share u64 | wrap_sign_share u64
  | extra_params [u32][u64..]
  | pred_meta (bit_order u8, sem u8, out_bytes u32) | cut_pred_meta (same)
  | coeff_meta (bit_order u8, sem u8)
  | pred_keys, cut_pred_keys, coeff_keys: each [u32 count]([u32 len][bytes])..
  | base_coeff_share [u32][u64..] | total_delta_share [u32][u64..]
  | triples [u32 n]({a, b, c} u64 each) x n | bit_triples [u32 n]({a, b, c} u8) x n

A key is a dict with those names; u64 vectors and triples are numpy arrays
(triples uint64 [n][3], bit triples uint8 [n][3]), key blobs bytes.  A short
buffer raises ValueError("composite tape truncated").
"""
import struct

import numpy as np

# proto::BitOrder and proto::ShareSemantics (include/proto/pfss_backend.hpp:18-23).
MSB_FIRST, LSB_FIRST = 0, 1
XOR_BYTES, ADD_U64 = 0, 1

_VECS_HEAD = ("r_in_share_vec", "r_out_share", "wrap_share")
_KEY_LISTS = ("pred_keys", "cut_pred_keys", "coeff_keys")


def empty_key():
    z = np.zeros(0, dtype=np.uint64)
    return {"r_in_share": 0, "r_in_share_vec": z, "r_out_share": z, "wrap_share": z,
            "r_hi_share": 0, "wrap_sign_share": 0, "extra_params": z,
            "pred_meta": (MSB_FIRST, XOR_BYTES, 1), "cut_pred_meta": (MSB_FIRST, XOR_BYTES, 1),
            "coeff_meta": (MSB_FIRST, ADD_U64),
            "pred_keys": [], "cut_pred_keys": [], "coeff_keys": [],
            "base_coeff_share": z, "total_delta_share": z,
            "triples": np.zeros((0, 3), dtype=np.uint64),
            "bit_triples": np.zeros((0, 3), dtype=np.uint8)}


def _u64vec(v):
    a = np.ascontiguousarray(np.asarray(v, dtype=np.uint64))
    return struct.pack("<I", a.size) + a.astype("<u8").tobytes()


def write_composite_tape(k):
    out = [struct.pack("<Q", int(k["r_in_share"]) & (2**64 - 1))]
    out += [_u64vec(k[name]) for name in _VECS_HEAD]
    out.append(struct.pack("<QQ", int(k["r_hi_share"]) & (2**64 - 1),
                           int(k["wrap_sign_share"]) & (2**64 - 1)))
    out.append(_u64vec(k["extra_params"]))
    for meta in ("pred_meta", "cut_pred_meta"):
        bo, sem, ob = k[meta]
        out.append(struct.pack("<BBI", bo, sem, ob))
    out.append(struct.pack("<BB", *k["coeff_meta"]))
    for name in _KEY_LISTS:
        keys = k[name]
        out.append(struct.pack("<I", len(keys)))
        for blob in keys:
            b = bytes(blob)
            out.append(struct.pack("<I", len(b)) + b)
    out.append(_u64vec(k["base_coeff_share"]))
    out.append(_u64vec(k["total_delta_share"]))
    t = np.ascontiguousarray(np.asarray(k["triples"], dtype=np.uint64).reshape(-1, 3))
    out.append(struct.pack("<I", t.shape[0]) + t.astype("<u8").tobytes())
    bt = np.ascontiguousarray(np.asarray(k["bit_triples"], dtype=np.uint8).reshape(-1, 3))
    out.append(struct.pack("<I", bt.shape[0]) + bt.tobytes())
    return b"".join(out)


class _Reader:
    def __init__(self, data):
        self.b = memoryview(bytes(data))
        self.p = 0

    def need(self, n):
        if len(self.b) - self.p < n:
            raise ValueError("composite tape truncated")

    def take(self, n):
        self.need(n)
        v = self.b[self.p:self.p + n]
        self.p += n
        return v

    def u8(self):
        return self.take(1)[0]

    def u32(self):
        return struct.unpack("<I", self.take(4))[0]

    def u64(self):
        return struct.unpack("<Q", self.take(8))[0]

    def u64vec(self):
        n = self.u32()
        self.need(8 * n)
        return np.frombuffer(self.take(8 * n), dtype="<u8").astype(np.uint64)


def read_composite_tape(data):
    r = _Reader(data)
    k = {"r_in_share": r.u64()}
    for name in _VECS_HEAD:
        k[name] = r.u64vec()
    k["r_hi_share"] = r.u64()
    k["wrap_sign_share"] = r.u64()
    k["extra_params"] = r.u64vec()
    r.need(2 + 4 + 2 + 4 + 2)
    for meta in ("pred_meta", "cut_pred_meta"):
        bo, sem = r.u8(), r.u8()
        k[meta] = (bo, sem, r.u32())
    k["coeff_meta"] = (r.u8(), r.u8())
    for name in _KEY_LISTS:
        cnt = r.u32()
        keys = []
        for _ in range(cnt):
            ln = r.u32()
            keys.append(bytes(r.take(ln)))
        k[name] = keys
    k["base_coeff_share"] = r.u64vec()
    k["total_delta_share"] = r.u64vec()
    n = r.u32()
    r.need(24 * n)
    k["triples"] = np.frombuffer(r.take(24 * n), dtype="<u8").astype(np.uint64).reshape(n, 3)
    n = r.u32()
    r.need(3 * n)
    k["bit_triples"] = np.frombuffer(r.take(3 * n), dtype=np.uint8).reshape(n, 3).copy()
    return k
