"""Private scratch of the shipped kernels (CPU, from the compiler's output).

Every kernel of libsuf_hip.so must report ScratchSize 0 except those that
suf_amd.build.SCRATCH_ALLOWED names.  The softmax block is named there
because its uniform pointers overflow the SGPR file and the compiler keeps the
overflow in VGPR lanes: the frame size is reported although no instruction
touches scratch memory, which the second test checks in its assembly."""
import os
import re
import subprocess

import pytest

from suf_amd import build


def test_resource_report_has_no_unexpected_scratch():
    res = build.kernel_resources()
    if not res:
        pytest.skip("libsuf_hip.so not built with the resource report")
    build.check_scratch(res)
    hot = ["dcf_eval_bit_kernel", "lut_keyed_kernel", "packed_keyed_kernel", "public_mfma_kernel",
           "beaver_mfma2_kernel", "gate_chain_kernel", "layernorm2_kernel", "trunc_eval_table_kernel"]
    for name in hot:
        ks = [k for k in res if name in k]
        assert ks, name
        for k in ks:
            assert int(res[k].get("ScratchSize [bytes/lane]", "0")) == 0, k


def test_softmax_block_has_no_scratch_instructions(tmp_path):
    try:
        cc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    src = os.path.join(build.CSRC, "blocks.hip")
    asm = str(tmp_path / "blocks.s")
    flags = [f for f in build.HIPCC_FLAGS if not f.startswith("-R") and f != "-fno-caret-diagnostics"]
    subprocess.run([cc] + flags + ["--cuda-device-only", "-S", src, "-o", asm], check=True,
                   stdout=subprocess.DEVNULL, stderr=subprocess.DEVNULL)
    text = open(asm).read()
    bodies = re.findall(r"^(_ZN\S*softmax2\S*kernel\S*):.*?\n(.*?)s_endpgm", text, flags=re.S | re.M)
    assert len(bodies) >= 3 and any("team" in name for name, _ in bodies)
    for name, body in bodies:
        assert not re.search(r"^\s+(scratch_|buffer_)", body, flags=re.M), name
        assert "v_writelane" in body  # the spill slots are VGPR lanes
