"""Writes tests/golden/dcf_myl7.json from the reference's own myl7 DCF
(third_party/myl7_fss/src/dcf.c + prg/aes128_mmo.c + group/{bytes,u128_le}.c
and include/proto/myl7_fss_backend.hpp, built unmodified by
oracle/build_ref.sh into oracle/_ref/).

Every key's correction words come from the reference dcf_gen with fixed
seeds and a fixed PRG state; every expected output comes from the reference
adapter's eval_dcf / eval_dcf_many_u64.  The blob layout
[in_bits][chunks][party][0][payload_len u32 LE] + [seed][cws][cw_np1] is the
adapter's (myl7_fss_backend.hpp:131-213).

Run from the repository root:  python tests/golden/make_golden.py
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as ol  # noqa: E402


def blob(in_bits, party, payload_len, seed, cws, np1):
    h = bytes([in_bits, 1, party, 0]) + payload_len.to_bytes(4, "little")
    return h + bytes(seed) + bytes(cws) + bytes(np1)


def main():
    if not ol.ref_available():
        raise SystemExit("oracle/_ref not built: run sh oracle/build_ref.sh first")
    cases = []
    for group, gname in ((ol.GROUP_XOR, "xor"), (ol.GROUP_ADD, "add")):
        ref = ol.ref_lib(group)
        state = ol.mt64_bytes(3, ol.PRG_STATE_BYTES)  # PRG state from mt19937_64(3)
        ref.ref_prg_init(ol.ptr(state), ol.PRG_STATE_BYTES)
        seed_words = ol.mt64(4, 4096)  # DCF seeds from mt19937_64(4)
        sb = (seed_words & np.uint64(0xFF)).astype(np.uint8)
        pos = 0
        for in_bits, plen, alphas in ((16, 1, [1, 0x8000, 0xFFFF, 12345]),
                                      (64, 1, [1, 2**63 + 5, 2**64 - 1, 0x0123456789ABCDEF]),
                                      (64, 8, [2**62 + 77]),
                                      (12, 16, [2049])):
            mask = (1 << in_bits) - 1
            for alpha in alphas:
                s0 = sb[pos:pos + 16].copy()
                s1 = sb[pos + 16:pos + 32].copy()
                pos += 32
                payload = bytes([(0x01 + 17 * k) & 0xFF for k in range(plen)])
                beta = np.zeros(16, dtype=np.uint8)
                beta[:plen] = np.frombuffer(payload, dtype=np.uint8)
                beta[15] &= 0x7F
                alpha_le = np.frombuffer(int(alpha).to_bytes(8, "little"), dtype=np.uint8).copy()
                cws = np.zeros(in_bits * 33, dtype=np.uint8)
                np1 = np.zeros(16, dtype=np.uint8)
                ref.ref_dcf_gen(in_bits, ol.ptr(alpha_le), ol.ptr(beta), ol.ptr(s0.copy()),
                                ol.ptr(s1.copy()), ol.ptr(cws), ol.ptr(np1))
                k0 = blob(in_bits, 0, plen, s0, cws, np1)
                k1 = blob(in_bits, 1, plen, s1, cws, np1)
                xs = sorted({(alpha + d) & mask for d in (-2, -1, 0, 1, 2)} |
                            {0, mask, int(seed_words[pos]) & mask})
                outs = {}
                for party, key in ((0, k0), (1, k1)):
                    kb = np.frombuffer(key, dtype=np.uint8).copy()
                    full = []
                    for x in xs:
                        buf = np.zeros(64, dtype=np.uint8)
                        n = ref.ref_adapter_eval(in_bits, ol.ptr(kb), len(kb), x, ol.ptr(buf), 64)
                        assert n == plen
                        full.append(buf[:plen].tobytes().hex())
                    flat = np.ascontiguousarray(np.tile(kb, (len(xs), 1)))
                    bits = np.zeros(len(xs), dtype=np.uint8)
                    xa = np.array(xs, dtype=np.uint64)
                    assert ref.ref_adapter_eval_many(in_bits, len(kb), ol.ptr(flat),
                                                     ol.ptr(xa, ol.u64p), len(xs), 1,
                                                     ol.ptr(bits)) == 0
                    outs[party] = {"full": full, "bit": [int(b) for b in bits]}
                cases.append({
                    "group": gname, "in_bits": in_bits, "alpha": str(alpha),
                    "payload": payload.hex(), "key0": k0.hex(), "key1": k1.hex(),
                    "xs": [str(x) for x in xs],
                    "out0": outs[0], "out1": outs[1],
                })
    doc = {
        "source": "reference myl7/fss v0.7.1 dcf.c + aes128_mmo.c (kBlocks=8, kLambda=16) "
                  "and proto::Myl7FssBackend, built by oracle/build_ref.sh",
        "prg_state": ol.mt64_bytes(3, ol.PRG_STATE_BYTES).tobytes().hex(),
        "cases": cases,
    }
    path = os.path.join(HERE, "dcf_myl7.json")
    with open(path, "w") as f:
        json.dump(doc, f, indent=1)
    print("wrote", path, len(cases), "cases")


if __name__ == "__main__":
    main()
