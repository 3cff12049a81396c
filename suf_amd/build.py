"""Builds libsuf_hip.so (gfx950) in-tree with hipcc.

    python -m suf_amd.build          # from the repository root

Each .hip translation unit under suf_amd/csrc is compiled to an object file
under suf_amd/lib/obj and linked into suf_amd/lib/libsuf_hip.so.  The build
always recompiles (it is the "does it build" check); pass --if-stale to skip
units whose object file is newer than every source and header.
"""
import argparse
import glob
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIBDIR = os.path.join(PKG, "lib")
OBJDIR = os.path.join(LIBDIR, "obj")
LIB = os.path.join(LIBDIR, "libsuf_hip.so")
ARCH = "gfx950"

HIPCC_FLAGS = [
    "--offload-arch=" + ARCH,
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-I" + os.path.join(ROOT, "include"),
    "-I" + CSRC,
    # Keep the compiler from emitting packed FP32 instructions.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Per-kernel register and private-segment report, checked below.
    "-Rpass-analysis=kernel-resource-usage", "-fno-caret-diagnostics",
]

# Kernels allowed a private segment, with the reason.  Every other kernel
# must report ScratchSize 0, or the build fails.
SCRATCH_ALLOWED = {
    # Dealer-side keygen (not on the online path): the four PRG blocks of a
    # level, indexed by the block loop, spill 144 bytes per lane.
    "dcf_gen_kernel": "dealer keygen",
    "trunc_gen_kernel": "dealer keygen",
    # SGPR spill slots only: the block's ~100 uniform pointers exceed the
    # SGPR file, and the compiler keeps the overflow in VGPR lanes
    # (v_writelane / v_readlane).  The frame size is reported, but the kernel
    # has no scratch memory instruction (tests/test_build_scratch.py).
    "softmax2_kernel": "SGPR spill slots in VGPR lanes, no scratch memory access",
    "softmax2_team_kernel": "SGPR spill slots in VGPR lanes, no scratch memory access",
}
RESOURCE_REPORT = os.path.join(LIBDIR, "kernel_resources.txt")


def hipcc():
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libsuf_hip.so)")


def _deps():
    return glob.glob(os.path.join(CSRC, "*.hpp")) + glob.glob(os.path.join(ROOT, "include", "*.h"))


def _stale(src, obj):
    if not os.path.exists(obj):
        return True
    t = os.path.getmtime(obj)
    return any(os.path.getmtime(p) > t for p in [src] + _deps())


def parse_resource_usage(text):
    """{kernel symbol: {field: value}} from -Rpass-analysis=kernel-resource-usage
    remarks (Function Name, VGPRs, AGPRs, ScratchSize, Occupancy, ...)."""
    out, cur = {}, None
    for line in text.splitlines():
        if "kernel-resource-usage" not in line:
            continue
        m = re.search(r"remark:\s+(.*?)\s*\[-Rpass-analysis", line)
        if not m:
            continue
        body = m.group(1)
        if body.startswith("Function Name:"):
            cur = body.split(":", 1)[1].strip()
            out[cur] = {}
        elif cur is not None and ":" in body:
            k, v = body.rsplit(":", 1)
            out[cur][k.strip()] = v.strip()
    return out


def _compile(args):
    cc, src, obj = args
    tmp = obj + ".tmp"
    cmd = [cc] + HIPCC_FLAGS + ["-c", src, "-o", tmp]
    r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if r.returncode != 0:
        out = "\n".join(l for l in r.stdout.splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError("hipcc failed for %s:\n%s" % (os.path.basename(src), out))
    out = "\n".join(l for l in r.stdout.splitlines()
                    if "packed-fp32-ops" not in l and "kernel-resource-usage" not in l)
    os.replace(tmp, obj)
    with open(obj + ".res", "w") as f:
        f.write(r.stdout)
    return out


def kernel_resources():
    """Resource report of every kernel in the last build (from the remarks
    each object's compile wrote next to it)."""
    res = {}
    for p in sorted(glob.glob(os.path.join(OBJDIR, "*.o.res"))):
        for k, v in parse_resource_usage(open(p).read()).items():
            v["file"] = os.path.basename(p)[:-len(".o.res")]
            res[k] = v
    return res


def scratch_allowed(symbol):
    return next((why for name, why in SCRATCH_ALLOWED.items() if name in symbol), None)


def check_scratch(res):
    """Fails on any kernel with a private segment that SCRATCH_ALLOWED does
    not name; writes the report to suf_amd/lib/kernel_resources.txt."""
    bad = []
    lines = []
    for k in sorted(res):
        v = res[k]
        sc = int(v.get("ScratchSize [bytes/lane]", "0"))
        why = scratch_allowed(k)
        lines.append("%-70s %-18s VGPR %4s AGPR %4s scratch %4d occupancy %s%s" % (
            k, v["file"], v.get("VGPRs", "?"), v.get("AGPRs", "?"), sc, v.get("Occupancy [waves/SIMD]", "?"),
            ("  (allowed: %s)" % why) if sc and why else ""))
        if sc and not why:
            bad.append("%s (%s): %d bytes/lane" % (k, v["file"], sc))
    with open(RESOURCE_REPORT, "w") as f:
        f.write("\n".join(lines) + "\n")
    if bad:
        raise RuntimeError("kernels with private scratch (see %s):\n  %s"
                           % (RESOURCE_REPORT, "\n  ".join(bad)))


def build(if_stale=False, jobs=None):
    cc = hipcc()
    os.makedirs(OBJDIR, exist_ok=True)
    srcs = sorted(glob.glob(os.path.join(CSRC, "*.hip")) + glob.glob(os.path.join(CSRC, "*.cpp")))
    work = []
    objs = []
    for s in srcs:
        o = os.path.join(OBJDIR, os.path.basename(s) + ".o")
        objs.append(o)
        if not if_stale or _stale(s, o):
            work.append((cc, s, o))
    jobs = jobs or min(8, max(1, os.cpu_count() or 1))
    with ThreadPoolExecutor(jobs) as ex:
        for out in ex.map(_compile, work):
            if out.strip():
                sys.stderr.write(out + "\n")
    if work or not os.path.exists(LIB):
        tmp = LIB + ".tmp"
        cmd = [cc, "--offload-arch=" + ARCH, "-shared", "-fPIC", "-o", tmp] + objs
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError("link failed:\n" + r.stdout)
        os.replace(tmp, LIB)
    check_scratch(kernel_resources())
    return LIB


HOST_SRC = os.path.join(PKG, "host")
CPP_TESTS = os.path.join(ROOT, "tests", "cpp")
CPP_TEST_OUT = os.path.join(CPP_TESTS, "_build")


def build_host_tests():
    """Compiles the C++ proto-interface backend (suf_amd/host) into each C++
    test driver under tests/cpp, linked against libsuf_hip.so (g++, no HIP
    headers: the backend reaches the GPU only through the C ABI)."""
    os.makedirs(CPP_TEST_OUT, exist_ok=True)
    host = sorted(glob.glob(os.path.join(HOST_SRC, "*.cpp")))
    outs = []
    for t in sorted(glob.glob(os.path.join(CPP_TESTS, "*.cpp"))):
        exe = os.path.join(CPP_TEST_OUT, os.path.splitext(os.path.basename(t))[0])
        rel = os.path.relpath(LIBDIR, CPP_TEST_OUT)
        cmd = ["g++", "-std=c++17", "-O2", "-Wall", "-Wextra", "-pthread",
               "-I" + os.path.join(ROOT, "include"), t] + host + [
               "-L" + LIBDIR, "-lsuf_hip", "-Wl,-rpath,$ORIGIN/" + rel,
               "-Wl,-rpath-link,/opt/rocm/lib", "-o", exe + ".tmp"]
        r = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
        if r.returncode != 0:
            raise RuntimeError("g++ failed for %s:\n%s" % (os.path.basename(t), r.stdout))
        os.replace(exe + ".tmp", exe)
        outs.append(exe)
    return outs


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--if-stale", action="store_true")
    ap.add_argument("-j", type=int, default=None)
    a = ap.parse_args()
    print(build(if_stale=a.if_stale, jobs=a.j))
    for exe in build_host_tests():
        print(exe)


if __name__ == "__main__":
    main()
